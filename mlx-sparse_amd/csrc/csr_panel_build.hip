// csr_panel_build.hip - builds the column-panel copy of a bound plan.
//
// Layout (the SpMV that reads it is in csr_panel.hip):
//   panels  x is cut into panels of PW = 128 KB / sizeof(accumulator)
//           entries (32768 for float32/float16/bfloat16, 16384 for
//           complex64): the widened panel fits in LDS.
//   tiles   consecutive short rows (the plan's rule: a row is long when it
//           holds more than W values; long rows stay on the row-block path)
//           grouped so that a tile's products plus one word per row fit in
//           TW = 64 KB / sizeof(accumulator) LDS words.  A short row starts a
//           tile at r = 0, after a long row, or when (indptr[r] + r) / H
//           changes, H = TW - W; every row start of a tile then lies in one
//           H-wide window of the word range and each row adds at most W + 1
//           words, so a tile holds at most H + W = TW words.
//   copy    the values of short rows whose column lies in [0, n_cols),
//           ordered by (panel, tile, stored position).  Segment (q, t) - the
//           values of tile t in panel q - starts at seg[q * n_tiles + t] and
//           is padded to a multiple of 4 entries (value 0, column 0, word
//           0xFFFF, which no tile has), so every segment starts on a 16-byte
//           boundary of the product buffer and pass 2 reads whole quads.
//           Each value keeps its column inside the panel (u16) and its LDS
//           word in the tile, dest = (p - first value of the tile) +
//           (row - first row of the tile) (u16): a row's values sit at
//           consecutive words in stored order, one spare word after each row.
//
// Construction on the device: per-row tile flags, a prefix sum (tile ids),
// per-value sort keys q * n_tiles + t (values dropped from the copy get the
// key n_panels * n_tiles, which sorts last), a stable radix sort of
// (key, position) pairs, segment starts by binary search over the sorted
// keys, padded starts by a prefix sum of the rounded lengths, then a
// gather of the values to their padded places.  The host reads two small arrays: the
// tile count and the panel boundaries, which size the copy and split pass 1
// into about one workgroup per CU.
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <vector>

#include "msx_device.h"
#include "msx_internal.h"

namespace msx {
namespace {

constexpr int kThreads = 256;
constexpr int64_t kMaxGrid = int64_t{1} << 20;
constexpr int64_t kPanelBytes = 131072;  // x panel in LDS during pass 1
constexpr int64_t kTileBytes = 65536;    // tile products in LDS during pass 2
constexpr int64_t kMaxPanels = 2048;
constexpr int64_t kMinChunk = 65536;     // values per pass-1 workgroup, about

uint32_t grid_for(int64_t n) {
  return static_cast<uint32_t>(std::max<int64_t>(1, std::min<int64_t>((n + kThreads - 1) / kThreads, kMaxGrid)));
}

int64_t acc_bytes(msx_vtype vt) { return vt == MSX_C64 ? 8 : 4; }

__device__ inline int64_t clamp64(int64_t v, int64_t lo, int64_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

// The plan's long-row rule (csr_plan.hip, classify): raw offsets, len > W.
template <class I>
__device__ inline bool row_long(const I *indptr, int64_t r, int64_t W) {
  return static_cast<int64_t>(indptr[r + 1]) - static_cast<int64_t>(indptr[r]) > W;
}

template <class I>
__device__ inline int64_t tile_key(const I *indptr, int64_t r, int64_t nnz, int64_t H) {
  return (clamp64(static_cast<int64_t>(indptr[r]), 0, nnz) + r) / H;
}

// flag[r] = 1 when short row r starts a tile; flag[n] = 0.
template <class I>
__global__ void __launch_bounds__(kThreads)
    tile_flags(const I *__restrict__ indptr, int64_t n, int64_t nnz, int64_t W, int64_t H,
               uint32_t *__restrict__ flag) {
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; r <= n;
       r += static_cast<int64_t>(gridDim.x) * kThreads) {
    bool f = false;
    if (r < n && !row_long(indptr, r, W))
      f = r == 0 || row_long(indptr, r - 1, W) ||
          tile_key(indptr, r, nnz, H) != tile_key(indptr, r - 1, nnz, H);
    flag[r] = f ? 1u : 0u;
  }
}

// tile_begin / tile_end from the flags and their exclusive prefix sum.
template <class I>
__global__ void __launch_bounds__(kThreads)
    tile_bounds(const I *__restrict__ indptr, int64_t n, int64_t W, const uint32_t *__restrict__ flag,
                const uint32_t *__restrict__ tid, int32_t *__restrict__ tile_begin,
                int32_t *__restrict__ tile_end) {
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; r < n;
       r += static_cast<int64_t>(gridDim.x) * kThreads) {
    if (row_long(indptr, r, W)) continue;
    const uint32_t t = tid[r] + flag[r] - 1u;
    if (flag[r]) tile_begin[t] = static_cast<int32_t>(r);
    if (r == n - 1 || row_long(indptr, r + 1, W) || flag[r + 1]) tile_end[t] = static_cast<int32_t>(r + 1);
  }
}

__global__ void __launch_bounds__(kThreads)
    fill_keys(int64_t nnz, uint32_t drop, uint32_t *__restrict__ key, uint32_t *__restrict__ pos) {
  for (int64_t p = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; p < nnz;
       p += static_cast<int64_t>(gridDim.x) * kThreads) {
    key[p] = drop;
    pos[p] = static_cast<uint32_t>(p);
  }
}

// One thread per short row: sort key and (column in panel | dest << 16) of
// each of its values.  Values with a column outside [0, n_cols) keep the
// drop key and are counted.
template <class I>
__global__ void __launch_bounds__(kThreads)
    panel_keys(const I *__restrict__ indices, const I *__restrict__ indptr, int64_t n, int64_t nnz,
               int64_t n_cols, int64_t W, int64_t PW, int64_t TW, uint32_t n_tiles,
               const uint32_t *__restrict__ flag, const uint32_t *__restrict__ tid,
               const int32_t *__restrict__ tile_begin, uint32_t *__restrict__ key,
               uint32_t *__restrict__ aux, unsigned long long *__restrict__ dropped) {
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; r < n;
       r += static_cast<int64_t>(gridDim.x) * kThreads) {
    if (row_long(indptr, r, W)) continue;
    const uint32_t t = tid[r] + flag[r] - 1u;
    const int64_t r0 = tile_begin[t];
    const int64_t b0 = clamp64(static_cast<int64_t>(indptr[r0]), 0, nnz);
    const int64_t s = clamp64(static_cast<int64_t>(indptr[r]), 0, nnz);
    const int64_t e = clamp64(static_cast<int64_t>(indptr[r + 1]), s, nnz);
    unsigned long long lost = 0;
    for (int64_t p = s; p < e; ++p) {
      const int64_t c = static_cast<int64_t>(indices[p]);
      const int64_t dest = (p - b0) + (r - r0);
      if (c >= 0 && c < n_cols && dest >= 0 && dest < TW) {
        const int64_t q = c / PW;
        key[p] = static_cast<uint32_t>(q * n_tiles + t);
        aux[p] = static_cast<uint32_t>(c - q * PW) | (static_cast<uint32_t>(dest) << 16);
      } else {
        ++lost;
      }
    }
    if (lost) atomicAdd(dropped, lost);
  }
}

// seg[k] = first index of the sorted keys >= k, for k in [0, n_keys].
__global__ void __launch_bounds__(kThreads)
    segment_starts(const uint32_t *__restrict__ sorted, int64_t nnz, int64_t n_keys,
                   uint32_t *__restrict__ seg) {
  for (int64_t k = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; k <= n_keys;
       k += static_cast<int64_t>(gridDim.x) * kThreads) {
    int64_t lo = 0, hi = nnz;  // first i with sorted[i] >= k
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (static_cast<int64_t>(sorted[mid]) < k) lo = mid + 1; else hi = mid;
    }
    seg[k] = static_cast<uint32_t>(lo);
  }
}

__global__ void __launch_bounds__(kThreads)
    panel_bounds(const uint32_t *__restrict__ seg, int64_t n_panels, int64_t n_tiles,
                 uint32_t *__restrict__ out) {
  for (int64_t q = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; q <= n_panels;
       q += static_cast<int64_t>(gridDim.x) * kThreads)
    out[q] = seg[q * n_tiles];
}

// len[k] = segment k's length rounded up to a multiple of 4; len[n_keys] = 0.
__global__ void __launch_bounds__(kThreads)
    padded_lengths(const uint32_t *__restrict__ seg, int64_t n_keys, uint32_t *__restrict__ len) {
  for (int64_t k = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; k <= n_keys;
       k += static_cast<int64_t>(gridDim.x) * kThreads)
    len[k] = k < n_keys ? (seg[k + 1] - seg[k] + 3u) & ~3u : 0u;
}

// Sorted value i (key k) goes to pseg[k] + (i - seg[k]).
template <class S>
__global__ void __launch_bounds__(kThreads)
    panel_gather(const S *__restrict__ data, const uint32_t *__restrict__ pos,
                 const uint32_t *__restrict__ sorted_key, const uint32_t *__restrict__ seg,
                 const uint32_t *__restrict__ pseg, const uint32_t *__restrict__ aux, int64_t n_kept,
                 int64_t n_keys, int64_t nnz, int64_t n_values, S *__restrict__ out_data,
                 uint16_t *__restrict__ out_col, uint16_t *__restrict__ out_dest) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n_kept;
       i += static_cast<int64_t>(gridDim.x) * kThreads) {
    const int64_t k = sorted_key[i];
    if (k >= n_keys) continue;
    const int64_t at = static_cast<int64_t>(pseg[k]) + (i - static_cast<int64_t>(seg[k]));
    if (at < 0 || at >= n_values) continue;
    const int64_t p = clamp64(pos[i], 0, nnz - 1);
    out_data[at] = data[p];
    const uint32_t a = aux[p];
    out_col[at] = static_cast<uint16_t>(a & 0xFFFFu);
    out_dest[at] = static_cast<uint16_t>(a >> 16);
  }
}

// Refresh of the copy's values after the matrix's values changed (same
// indices and indptr): one workgroup per tile.  The tile's rows fill a map
// from LDS word to (row - first row of the tile); an entry with word d then
// came from position b0 + d - map[d], the inverse of dest = (p - b0) +
// (row - r0).  Every panel's segment of the tile is regathered; padding
// entries (word 0xFFFF, outside every tile) keep their zero.
template <class S, class I>
__global__ void __launch_bounds__(kThreads)
    panel_refresh(const S *__restrict__ data, const I *__restrict__ indptr, int64_t nnz,
                  const int32_t *__restrict__ tile_begin, const int32_t *__restrict__ tile_end,
                  const uint32_t *__restrict__ seg, int64_t n_panels, int64_t n_tiles, int64_t TW,
                  const uint16_t *__restrict__ dest, S *__restrict__ out) {
  __shared__ uint16_t row_of[kTileBytes / 4];  // TW <= 16384 words
  const int64_t t = blockIdx.x;
  const int64_t r0 = tile_begin[t], r1 = tile_end[t];
  const int64_t b0 = clamp64(static_cast<int64_t>(indptr[r0]), 0, nnz);
  for (int64_t r = r0 + threadIdx.x; r < r1; r += kThreads) {
    const int64_t s = clamp64(static_cast<int64_t>(indptr[r]), 0, nnz);
    const int64_t e = clamp64(static_cast<int64_t>(indptr[r + 1]), s, nnz);
    for (int64_t p = s; p < e; ++p) {
      const int64_t w = (p - b0) + (r - r0);
      if (w >= 0 && w < TW) row_of[w] = static_cast<uint16_t>(r - r0);
    }
  }
  __syncthreads();
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  for (int64_t q = wave; q < n_panels; q += kThreads / kWave) {
    const int64_t a = seg[q * n_tiles + t], b = seg[q * n_tiles + t + 1];
    for (int64_t e = a + lane; e < b; e += kWave) {
      const int64_t d = dest[e];
      if (d >= TW) continue;
      out[e] = data[clamp64(b0 + d - row_of[d], 0, nnz - 1)];
    }
  }
}

int bits_for(uint64_t v) {
  int b = 0;
  while (b < 64 && (v >> b) != 0) ++b;
  return std::max(1, b);
}

size_t round256(size_t b) { return (b + 255) / 256 * 256; }

// Device scratch of the build, released on every exit path.
struct Scratch {
  std::vector<void *> ptrs;
  hipStream_t stream;
  ~Scratch() {
    (void)hipStreamSynchronize(stream);
    for (void *p : ptrs) (void)hipFree(p);
  }
  template <class T>
  bool alloc(T **out, size_t bytes) {
    void *p = nullptr;
    if (hipMalloc(&p, std::max<size_t>(bytes, 256)) != hipSuccess) {
      (void)hipGetLastError();
      return false;
    }
    ptrs.push_back(p);
    *out = static_cast<T *>(p);
    return true;
  }
};

msx_status no_memory() {
  return fail(MSX_ENOMEM, "msx_csr_plan_create_bound: device allocation of the panel copy failed.");
}

template <class V, class I>
msx_status build_typed(msx_csr_plan *p, const void *data_v, const void *indices_v,
                       const void *indptr_v, hipStream_t stream) {
  using S = typename V::Storage;
  using A = typename V::Acc;
  const auto *data = static_cast<const S *>(data_v);
  const auto *indices = static_cast<const I *>(indices_v);
  const auto *indptr = static_cast<const I *>(indptr_v);
  const int64_t n = p->n_rows, nnz = p->nnz, W = p->block_nnz;
  const int64_t PW = kPanelBytes / static_cast<int64_t>(sizeof(A));
  const int64_t TW = kTileBytes / static_cast<int64_t>(sizeof(A));
  const int64_t H = TW - W;
  const int64_t P = (p->n_cols + PW - 1) / PW;
  Scratch tmp{{}, stream};

  // Tiles.
  uint32_t *flag = nullptr, *tid = nullptr;
  if (!tmp.alloc(&flag, sizeof(uint32_t) * (n + 1)) || !tmp.alloc(&tid, sizeof(uint32_t) * (n + 1)))
    return no_memory();
  hipLaunchKernelGGL((tile_flags<I>), dim3(grid_for(n + 1)), dim3(kThreads), 0, stream, indptr, n,
                     nnz, W, H, flag);
  MSX_HIP_TRY(hipGetLastError());
  size_t scan_bytes = 0;
  MSX_HIP_TRY(hipcub::DeviceScan::ExclusiveSum(nullptr, scan_bytes, flag, tid, static_cast<int>(n + 1), stream));
  void *scan_tmp = nullptr;
  if (!tmp.alloc(&scan_tmp, scan_bytes)) return no_memory();
  MSX_HIP_TRY(hipcub::DeviceScan::ExclusiveSum(scan_tmp, scan_bytes, flag, tid, static_cast<int>(n + 1), stream));
  uint32_t n_tiles_u = 0;
  MSX_HIP_TRY(hipMemcpyAsync(&n_tiles_u, tid + n, sizeof(uint32_t), hipMemcpyDeviceToHost, stream));
  MSX_HIP_TRY(hipStreamSynchronize(stream));
  const int64_t n_tiles = n_tiles_u;
  if (n_tiles == 0) return MSX_OK;
  const int64_t n_keys = P * n_tiles;  // also the drop key
  if (n_keys + 1 >= (int64_t{1} << 32))
    return fail(MSX_EINVAL, "msx_csr_plan_create_bound: too many panel segments for 32-bit keys.");

  // Per-plan metadata: tiles, segment starts, pass-1 chunks (at most
  // P + CUs + 1 of them, see below).
  int cus = 0;
  MSX_HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, p->device));
  cus = std::max(cus, 1);
  const int64_t max_chunks = P + cus + 1;
  const size_t b_tb = round256(sizeof(int32_t) * n_tiles);
  const size_t b_seg = round256(sizeof(uint32_t) * (n_keys + 1));
  const size_t b_cb = round256(sizeof(int64_t) * (max_chunks + 1));
  const size_t b_cp = round256(sizeof(int32_t) * max_chunks);
  char *meta = nullptr;
  if (hipMalloc(&meta, 2 * b_tb + b_seg + b_cb + b_cp) != hipSuccess) {
    (void)hipGetLastError();
    return no_memory();
  }
  p->pn_meta = meta;
  p->pn_bytes = 2 * b_tb + b_seg + b_cb + b_cp;
  p->pn_tile_begin = reinterpret_cast<int32_t *>(meta);
  p->pn_tile_end = reinterpret_cast<int32_t *>(meta + b_tb);
  p->pn_seg = reinterpret_cast<uint32_t *>(meta + 2 * b_tb);
  p->pn_chunk_begin = reinterpret_cast<int64_t *>(meta + 2 * b_tb + b_seg);
  p->pn_chunk_panel = reinterpret_cast<int32_t *>(meta + 2 * b_tb + b_seg + b_cb);
  hipLaunchKernelGGL((tile_bounds<I>), dim3(grid_for(n)), dim3(kThreads), 0, stream, indptr, n, W, flag,
                     tid, p->pn_tile_begin, p->pn_tile_end);
  MSX_HIP_TRY(hipGetLastError());

  // Keys, stable sort, segment starts.
  uint32_t *key = nullptr, *key_out = nullptr, *pos = nullptr, *pos_out = nullptr, *aux = nullptr;
  unsigned long long *dropped = nullptr;
  const size_t b_nnz = sizeof(uint32_t) * std::max<int64_t>(nnz, 1);
  if (!tmp.alloc(&key, b_nnz) || !tmp.alloc(&key_out, b_nnz) || !tmp.alloc(&pos, b_nnz) ||
      !tmp.alloc(&pos_out, b_nnz) || !tmp.alloc(&aux, b_nnz) || !tmp.alloc(&dropped, sizeof(*dropped)))
    return no_memory();
  MSX_HIP_TRY(hipMemsetAsync(dropped, 0, sizeof(*dropped), stream));
  hipLaunchKernelGGL(fill_keys, dim3(grid_for(nnz)), dim3(kThreads), 0, stream, nnz,
                     static_cast<uint32_t>(n_keys), key, pos);
  MSX_HIP_TRY(hipGetLastError());
  hipLaunchKernelGGL((panel_keys<I>), dim3(grid_for(n)), dim3(kThreads), 0, stream, indices, indptr, n,
                     nnz, p->n_cols, W, PW, TW, static_cast<uint32_t>(n_tiles), flag, tid,
                     p->pn_tile_begin, key, aux, dropped);
  MSX_HIP_TRY(hipGetLastError());
  const int end_bit = bits_for(static_cast<uint64_t>(n_keys));
  size_t sort_bytes = 0;
  MSX_HIP_TRY(hipcub::DeviceRadixSort::SortPairs(nullptr, sort_bytes, key, key_out, pos, pos_out,
                                                 static_cast<int>(nnz), 0, end_bit, stream));
  void *sort_tmp = nullptr;
  if (!tmp.alloc(&sort_tmp, sort_bytes)) return no_memory();
  MSX_HIP_TRY(hipcub::DeviceRadixSort::SortPairs(sort_tmp, sort_bytes, key, key_out, pos, pos_out,
                                                 static_cast<int>(nnz), 0, end_bit, stream));
  uint32_t *seg_raw = nullptr, *plen = nullptr;
  if (!tmp.alloc(&seg_raw, sizeof(uint32_t) * (n_keys + 1)) ||
      !tmp.alloc(&plen, sizeof(uint32_t) * (n_keys + 1)))
    return no_memory();
  hipLaunchKernelGGL(segment_starts, dim3(grid_for(n_keys + 1)), dim3(kThreads), 0, stream, key_out,
                     nnz, n_keys, seg_raw);
  MSX_HIP_TRY(hipGetLastError());
  hipLaunchKernelGGL(padded_lengths, dim3(grid_for(n_keys + 1)), dim3(kThreads), 0, stream, seg_raw,
                     n_keys, plen);
  MSX_HIP_TRY(hipGetLastError());
  size_t pscan_bytes = 0;
  MSX_HIP_TRY(hipcub::DeviceScan::ExclusiveSum(nullptr, pscan_bytes, plen, p->pn_seg,
                                               static_cast<int>(n_keys + 1), stream));
  void *pscan_tmp = nullptr;
  if (!tmp.alloc(&pscan_tmp, pscan_bytes)) return no_memory();
  MSX_HIP_TRY(hipcub::DeviceScan::ExclusiveSum(pscan_tmp, pscan_bytes, plen, p->pn_seg,
                                               static_cast<int>(n_keys + 1), stream));
  uint32_t n_kept_u = 0;
  MSX_HIP_TRY(hipMemcpyAsync(&n_kept_u, seg_raw + n_keys, sizeof(uint32_t), hipMemcpyDeviceToHost, stream));
  uint32_t *pbound = nullptr;
  if (!tmp.alloc(&pbound, sizeof(uint32_t) * (P + 1))) return no_memory();
  hipLaunchKernelGGL(panel_bounds, dim3(grid_for(P + 1)), dim3(kThreads), 0, stream, p->pn_seg, P,
                     n_tiles, pbound);
  MSX_HIP_TRY(hipGetLastError());
  std::vector<uint32_t> pb(static_cast<size_t>(P + 1));
  unsigned long long lost = 0;
  MSX_HIP_TRY(hipMemcpyAsync(pb.data(), pbound, sizeof(uint32_t) * (P + 1), hipMemcpyDeviceToHost, stream));
  MSX_HIP_TRY(hipMemcpyAsync(&lost, dropped, sizeof(lost), hipMemcpyDeviceToHost, stream));
  MSX_HIP_TRY(hipStreamSynchronize(stream));
  const int64_t n_values = pb[P];
  const int64_t n_kept = n_kept_u;

  // Pass-1 chunks: about one per CU (C in total, at least kMinChunk values
  // each), never across a panel boundary.  Panel q gets round(C * len / total)
  // chunks, at least one: a panel holding a few values more than its share
  // must not add a chunk, or the grid spills into a second, nearly empty
  // round of workgroups.  The total stays within C + P / 2 + 1 <= CUs + P.
  const int64_t C = std::max<int64_t>(1, std::min<int64_t>(cus, n_values / kMinChunk));
  std::vector<int64_t> cbeg;
  std::vector<int32_t> cpan;
  for (int64_t q = 0; q < P; ++q) {
    const int64_t a = pb[q], b = pb[q + 1];
    if (b <= a) continue;
    const int64_t c = std::max<int64_t>(1, (2 * C * (b - a) + n_values) / (2 * n_values));
    for (int64_t i = 0; i < c; ++i) {
      cbeg.push_back(a + (((b - a) * i / c) & ~int64_t{3}));
      cpan.push_back(static_cast<int32_t>(q));
    }
  }
  cbeg.push_back(n_values);
  const int64_t n_chunks = static_cast<int64_t>(cpan.size());
  if (n_chunks > max_chunks) return fail(MSX_EINVAL, "msx_csr_plan_create_bound: panel chunk table overflow.");

  // The copy and its product buffer.
  const size_t b_data = round256(sizeof(S) * std::max<int64_t>(n_values, 1));
  const size_t b_u16 = round256(sizeof(uint16_t) * std::max<int64_t>(n_values, 1));
  const size_t b_prod = round256(sizeof(A) * std::max<int64_t>(n_values, 1));
  char *base = nullptr;
  if (hipMalloc(&base, b_data + 2 * b_u16 + b_prod) != hipSuccess) {
    (void)hipGetLastError();
    return no_memory();
  }
  p->pn_base = base;
  p->pn_bytes += b_data + 2 * b_u16 + b_prod;
  p->pn_data = base;
  p->pn_col = reinterpret_cast<uint16_t *>(base + b_data);
  p->pn_dest = reinterpret_cast<uint16_t *>(base + b_data + b_u16);
  p->pn_prod = base + b_data + 2 * b_u16;
  // Padding entries: value 0, column 0, word 0xFFFF.
  MSX_HIP_TRY(hipMemsetAsync(p->pn_data, 0, b_data, stream));
  MSX_HIP_TRY(hipMemsetAsync(p->pn_col, 0, b_u16, stream));
  MSX_HIP_TRY(hipMemsetAsync(p->pn_dest, 0xFF, b_u16, stream));
  hipLaunchKernelGGL((panel_gather<S>), dim3(grid_for(n_kept)), dim3(kThreads), 0, stream, data,
                     pos_out, key_out, seg_raw, p->pn_seg, aux, n_kept, n_keys, nnz, n_values,
                     static_cast<S *>(p->pn_data), p->pn_col, p->pn_dest);
  MSX_HIP_TRY(hipGetLastError());
  MSX_HIP_TRY(hipMemcpyAsync(p->pn_chunk_begin, cbeg.data(), sizeof(int64_t) * cbeg.size(),
                             hipMemcpyHostToDevice, stream));
  MSX_HIP_TRY(hipMemcpyAsync(p->pn_chunk_panel, cpan.data(), sizeof(int32_t) * cpan.size(),
                             hipMemcpyHostToDevice, stream));
  MSX_HIP_TRY(hipStreamSynchronize(stream));
  p->n_panels = P;
  p->panel_width = PW;
  p->n_tiles = n_tiles;
  p->tile_words = TW;
  p->pn_values = n_values;
  p->pn_chunks = n_chunks;
  p->pn_dropped = lost != 0;
  return prepare_spmv_panels(p);
}

template <class V, class I>
msx_status refresh_typed(msx_csr_plan *p, const void *data, hipStream_t stream) {
  using S = typename V::Storage;
  if (p->n_tiles == 0 || p->pn_values == 0) return MSX_OK;
  hipLaunchKernelGGL((panel_refresh<S, I>), dim3(static_cast<uint32_t>(p->n_tiles)), dim3(kThreads), 0,
                     stream, static_cast<const S *>(data), static_cast<const I *>(p->indptr), p->nnz,
                     p->pn_tile_begin, p->pn_tile_end, p->pn_seg, p->n_panels, p->n_tiles,
                     p->tile_words, p->pn_dest, static_cast<S *>(p->pn_data));
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

}  // namespace

int64_t panels_min_values(int device) {
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) {
    (void)hipGetLastError();
    cus = 256;
  }
  return static_cast<int64_t>(std::max(cus, 1)) * kMinChunk;
}

bool panels_eligible(const msx_csr_plan *p) {
  if (p->n_cols < 1 || p->n_rows < 1 || p->nnz < 1 || p->nnz >= (int64_t{1} << 31) - 1) return false;
  const int64_t a = acc_bytes(p->vtype);
  const int64_t PW = kPanelBytes / a, TW = kTileBytes / a, H = TW - p->block_nnz;
  const int64_t P = (p->n_cols + PW - 1) / PW;
  if (P > kMaxPanels || H <= 0) return false;
  // Tiles: key windows of the word range, plus one break per long row.
  const int64_t tiles_max = (p->nnz + p->n_rows) / H + 2 + p->n_long;
  // Segment keys and padded copy offsets are 32-bit.
  return P * tiles_max + 1 < (int64_t{1} << 32) && p->nnz + 3 * P * tiles_max < (int64_t{1} << 32);
}

msx_status build_panels(msx_csr_plan *p, const void *data, const void *indices, const void *indptr,
                        hipStream_t stream) {
  switch (p->vtype) {
  case MSX_F32: return build_v<F32>(p, data, indices, indptr, stream);
  case MSX_F16: return build_v<F16>(p, data, indices, indptr, stream);
  case MSX_BF16: return build_v<BF16>(p, data, indices, indptr, stream);
  case MSX_C64: return build_v<C64>(p, data, indices, indptr, stream);
  }
  return fail(MSX_ETYPE, "msx_csr_plan_create_bound unsupported value dtype.");
}

msx_status refresh_panels(msx_csr_plan *p, const void *data, hipStream_t stream) {
  switch (p->vtype) {
  case MSX_F32: return refresh_v<F32>(p, data, stream);
  case MSX_F16: return refresh_v<F16>(p, data, stream);
  case MSX_BF16: return refresh_v<BF16>(p, data, stream);
  case MSX_C64: return refresh_v<C64>(p, data, stream);
  }
  return fail(MSX_ETYPE, "msx_csr_plan_refresh unsupported value dtype.");
}

}  // namespace msx
