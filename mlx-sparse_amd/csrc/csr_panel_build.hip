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

#define MSX_TRY_STATUS(expr)     \
  do {                           \
    msx_status _s = (expr);      \
    if (_s != MSX_OK) return _s; \
  } while (0)

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

// Virtual rows.  A row is long when it holds more than W values (the
// row-block plan's rule, csr_plan.hip classify: raw offsets, len > W).  A
// short row is one virtual row; a long row with its values clamped to
// [s, e) is max(1, ceil((e - s) / C)) virtual rows of C = min(W, 64)
// values (the last one shorter).  Every virtual row then holds at most W
// values, and a chunk, summed by one thread of pass 2, at most 64.
constexpr int64_t kLongChunk = 64;

__host__ __device__ inline int64_t long_chunk(int64_t W) { return W < kLongChunk ? W : kLongChunk; }

template <class I>
__device__ inline int64_t virtual_count(const I *indptr, int64_t r, int64_t nnz, int64_t W) {
  const int64_t b = static_cast<int64_t>(indptr[r]);
  const int64_t e = static_cast<int64_t>(indptr[r + 1]);
  if (e - b <= W) return 1;
  const int64_t C = long_chunk(W);
  const int64_t cs = clamp64(b, 0, nnz);
  const int64_t ce = clamp64(e, cs, nnz);
  return std::max<int64_t>(1, (ce - cs + C - 1) / C);
}

// count[r] = virtual rows of row r; count[n] = 0.
template <class I>
__global__ void __launch_bounds__(kThreads)
    vrow_counts(const I *__restrict__ indptr, int64_t n, int64_t nnz, int64_t W,
                uint32_t *__restrict__ count) {
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; r <= n;
       r += static_cast<int64_t>(gridDim.x) * kThreads)
    count[r] = r < n ? static_cast<uint32_t>(virtual_count(indptr, r, nnz, W)) : 0u;
}

// vstart / vslot of the virtual rows of row r (vbase: exclusive prefix of
// the counts); vstart[n_v] = clamped indptr[n].
template <class I>
__global__ void __launch_bounds__(kThreads)
    vrow_fill(const I *__restrict__ indptr, int64_t n, int64_t nnz, int64_t W,
              const uint32_t *__restrict__ vbase, uint32_t *__restrict__ vstart,
              int32_t *__restrict__ vslot) {
  const int64_t C = long_chunk(W);
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; r <= n;
       r += static_cast<int64_t>(gridDim.x) * kThreads) {
    const int64_t v = vbase[r];
    const int64_t s = clamp64(static_cast<int64_t>(indptr[r]), 0, nnz);
    if (r == n) {
      vstart[v] = static_cast<uint32_t>(s);
      continue;
    }
    const int64_t c = vbase[r + 1] - v;
    const bool is_long = static_cast<int64_t>(indptr[r + 1]) - static_cast<int64_t>(indptr[r]) > W;
    for (int64_t k = 0; k < c; ++k) {
      vstart[v + k] = static_cast<uint32_t>(std::min<int64_t>(s + k * C, nnz));
      vslot[v + k] = static_cast<int32_t>(is_long ? -1 - r : r);
    }
  }
}

// Row-pointer value of virtual row v clamped to [0, nnz]: indptr when the
// virtual rows are the rows, vstart otherwise.
template <class RP>
__device__ inline int64_t vpos(const RP *rowptr, int64_t v, int64_t nnz) {
  return clamp64(static_cast<int64_t>(rowptr[v]), 0, nnz);
}

template <class RP>
__device__ inline int64_t tile_key(const RP *rowptr, int64_t v, int64_t nnz, int64_t H) {
  return (vpos(rowptr, v, nnz) + v) / H;
}

// flag[v] = 1 when virtual row v starts a tile; flag[n_v] = 0.
template <class RP>
__global__ void __launch_bounds__(kThreads)
    tile_flags(const RP *__restrict__ rowptr, int64_t nv, int64_t nnz, int64_t H,
               uint32_t *__restrict__ flag) {
  for (int64_t v = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; v <= nv;
       v += static_cast<int64_t>(gridDim.x) * kThreads) {
    bool f = false;
    if (v < nv) f = v == 0 || tile_key(rowptr, v, nnz, H) != tile_key(rowptr, v - 1, nnz, H);
    flag[v] = f ? 1u : 0u;
  }
}

// tile_begin / tile_end from the flags and their exclusive prefix sum.
__global__ void __launch_bounds__(kThreads)
    tile_bounds(int64_t nv, const uint32_t *__restrict__ flag, const uint32_t *__restrict__ tid,
                int32_t *__restrict__ tile_begin, int32_t *__restrict__ tile_end) {
  for (int64_t v = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; v < nv;
       v += static_cast<int64_t>(gridDim.x) * kThreads) {
    const uint32_t t = tid[v] + flag[v] - 1u;
    if (flag[v]) tile_begin[t] = static_cast<int32_t>(v);
    if (v == nv - 1 || flag[v + 1]) tile_end[t] = static_cast<int32_t>(v + 1);
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

// One thread per virtual row: sort key and (column in panel | dest << 16)
// of each of its values.  Values with a column outside [0, n_cols) keep
// the drop key and are counted.
template <class I, class RP>
__global__ void __launch_bounds__(kThreads)
    panel_keys(const I *__restrict__ indices, const RP *__restrict__ rowptr, int64_t nv,
               int64_t nnz, int64_t n_cols, int64_t PW, int64_t TW, uint32_t n_tiles,
               const uint32_t *__restrict__ flag, const uint32_t *__restrict__ tid,
               const int32_t *__restrict__ tile_begin, uint32_t *__restrict__ key,
               uint32_t *__restrict__ aux, unsigned long long *__restrict__ dropped) {
  for (int64_t v = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; v < nv;
       v += static_cast<int64_t>(gridDim.x) * kThreads) {
    const uint32_t t = tid[v] + flag[v] - 1u;
    const int64_t v0 = tile_begin[t];
    const int64_t b0 = vpos(rowptr, v0, nnz);
    const int64_t s = vpos(rowptr, v, nnz);
    const int64_t e = clamp64(static_cast<int64_t>(rowptr[v + 1]), s, nnz);
    unsigned long long lost = 0;
    for (int64_t p = s; p < e; ++p) {
      const int64_t c = static_cast<int64_t>(indices[p]);
      const int64_t dest = (p - b0) + (v - v0);
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
// indices and indptr): one workgroup per tile, two per CU.  The tile's
// values are one contiguous range [b0, b1) of the matrix (at most TW of
// them), so they are first copied into LDS with coalesced dword loads
// through a descriptor (no branch per load).  Each virtual row v of the
// tile leaves a spare word after its values, dest = (p - b0) + (v - v0), so
// a bitmap of those gap words (one bit per LDS word, set by the rows) and
// the gaps before each 64-bit word of it (a prefix scan) give each word's
// position: p - b0 = d - (gaps below d).  The values are then spread in
// place from their positions to their words, so that a panel entry reads
// its value at its word d.  Every panel's segment of the tile is rewritten
// in quads (segments are padded to multiples of 4 entries): 4 words in one
// 8-byte load, 4 values in one store; padding entries (word 0xFFFF, outside
// every tile) get zero, as the build gave them.  LDS: the values, the
// bitmap and its prefix (refresh_lds_bytes).
constexpr int kRefreshUnroll = 4;
constexpr int kRefreshThreads = 1024;  // 16 waves; two workgroups per CU
constexpr int kRefreshWaves = kRefreshThreads / kWave;
constexpr int kRefreshPanels = 4;      // panel segments per wave whose loads are in flight

__host__ __device__ inline int64_t refresh_vals_bytes(int64_t TW, int64_t value_bytes) {
  return (TW * value_bytes + 16 + 15) / 16 * 16;  // + the start's offset inside a dword
}
__host__ __device__ inline int64_t refresh_lds_bytes(int64_t TW, int64_t value_bytes) {
  const int64_t nb = TW / 64;
  return refresh_vals_bytes(TW, value_bytes) + nb * 8 + nb * 4 + kRefreshWaves * 4;
}

template <class S>
struct alignas(4 * sizeof(S)) RefreshQuad {
  S v[4];
};

// held to 64 registers: two workgroups (eight waves per SIMD) per CU
template <class S, class RP>
__global__ void __launch_bounds__(kRefreshThreads) __attribute__((amdgpu_waves_per_eu(8, 8)))
    panel_refresh(const S *__restrict__ data, const RP *__restrict__ rowptr, int64_t nnz,
                  const int32_t *__restrict__ tile_begin, const int32_t *__restrict__ tile_end,
                  const uint32_t *__restrict__ seg, int64_t n_panels, int64_t n_tiles,
                  const uint16_t *__restrict__ dest, S *__restrict__ out) {
  // the tile's LDS words: 64 KB of accumulators (8-byte values: complex64)
  constexpr int kRefreshWords = static_cast<int>(kTileBytes / (sizeof(S) == 8 ? 8 : 4));
  constexpr int64_t TW = kRefreshWords;
  extern __shared__ __align__(16) unsigned char lds_raw[];
  unsigned char *vals = lds_raw;
  const int nbw = static_cast<int>(TW / 64);  // bitmap words (TW is a multiple of 64, <= 65536)
  auto *gap = reinterpret_cast<unsigned long long *>(lds_raw + refresh_vals_bytes(TW, sizeof(S)));
  auto *before = reinterpret_cast<uint32_t *>(gap + nbw);
  uint32_t *wsum = before + nbw;
  const int64_t t = blockIdx.x;
  const int64_t v0 = tile_begin[t], v1 = tile_end[t];
  const int64_t b0 = vpos(rowptr, v0, nnz);
  const int64_t b1 = clamp64(vpos(rowptr, v1, nnz), b0, b0 + TW);
  for (int i = threadIdx.x; i < nbw; i += kRefreshThreads) gap[i] = 0;
  // values [b0, b1) as the dwords that hold them: byte `off0` of the first
  // dword is position b0 (16-bit values may start mid-dword)
  const uintptr_t a0 = reinterpret_cast<uintptr_t>(data + b0);
  const uint32_t off0 = static_cast<uint32_t>(a0 & 3u);
  const uint32_t n_dw =
      static_cast<uint32_t>((off0 + static_cast<uint64_t>(b1 - b0) * sizeof(S) + 3) / 4);
  const auto r = make_rsrc(reinterpret_cast<const void *>(a0 - off0), uint64_t{4} * n_dw);
  auto *vw = reinterpret_cast<uint32_t *>(vals);
  // The whole dwords of the tile's values in 16-byte loads, all issued
  // before the first is used (kRefreshUnroll per thread cover TW values of
  // up to 8 bytes); the last n_dw % 4 dwords in dword loads.
  const uint32_t n_q = n_dw / 4;
  u32x4 w[kRefreshUnroll];
#pragma unroll
  for (int u = 0; u < kRefreshUnroll; ++u) {
    const uint32_t qi = threadIdx.x + u * kRefreshThreads;
    w[u] = qi < n_q ? BufLoad<16, kCacheStream>::load(r, 16u * qi) : u32x4{{0u, 0u, 0u, 0u}};
  }
  const uint32_t tail_i = 4 * n_q + threadIdx.x;
  const uint32_t tail = tail_i < n_dw ? __builtin_amdgcn_raw_buffer_load_b32(r, 4u * tail_i, 0, 0) : 0u;
  __syncthreads();  // the bitmap is clear
  for (int64_t v = v0 + threadIdx.x; v < v1; v += kRefreshThreads) {
    const int64_t s = vpos(rowptr, v, nnz);
    const int64_t e = clamp64(static_cast<int64_t>(rowptr[v + 1]), s, nnz);
    const int64_t g = (e - b0) + (v - v0);  // the row's spare word
    if (g >= 0 && g < TW) atomicOr(&gap[g >> 6], 1ull << (g & 63));
  }
#pragma unroll
  for (int u = 0; u < kRefreshUnroll; ++u) {
    const uint32_t qi = threadIdx.x + u * kRefreshThreads;
    if (qi < n_q) reinterpret_cast<u32x4 *>(vw)[qi] = w[u];
  }
  if (tail_i < n_dw) vw[tail_i] = tail;
  __syncthreads();
  {  // gaps before each bitmap word: a wave scan, then the wave totals in order
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int k = static_cast<int>(threadIdx.x);
    const uint32_t c = k < nbw ? static_cast<uint32_t>(__popcll(gap[k])) : 0u;
    uint32_t incl = c;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const uint32_t u = __shfl_up(incl, d, kWave);
      if (lane >= d) incl += u;
    }
    if (lane == kWave - 1) wsum[wave] = incl;
    __syncthreads();
    uint32_t off = 0;
    for (int w = 0; w < wave; ++w) off += wsum[w];
    if (k < nbw) before[k] = off + incl - c;
    __syncthreads();
  }
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int64_t nb = b1 - b0;
  {
    // The values are spread to their words: thread t takes the WPT
    // consecutive words from t * WPT (all in one bitmap word); value word i
    // of them holds the value at position (t * WPT + i) - (gaps below it),
    // so the chunk's values are one run of consecutive positions.  Every run
    // is read before any word is written (the words overlay the positions);
    // gap words get zero.
    constexpr int WPT = kRefreshWords / kRefreshThreads;  // 16, or 8 for 8-byte values
    const int w0 = static_cast<int>(threadIdx.x) * WPT;
    const int k = w0 >> 6, sh = w0 & 63;
    const unsigned long long bits = gap[k];
    const uint32_t cbits = static_cast<uint32_t>((bits >> sh) & ((1ull << WPT) - 1ull));
    int64_t pp = static_cast<int64_t>(w0) - before[k] - __popcll(bits & ((1ull << sh) - 1ull));
    RefreshQuad<S> wq[WPT / 4];
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
      S v{};
      if (!((cbits >> i) & 1u)) {
        if (pp >= 0 && pp < nb) __builtin_memcpy(&v, vals + off0 + pp * sizeof(S), sizeof(S));
        ++pp;
      }
      wq[i / 4].v[i % 4] = v;
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < WPT / 4; ++u) reinterpret_cast<RefreshQuad<S> *>(vals)[threadIdx.x * (WPT / 4) + u] = wq[u];
    __syncthreads();
  }
  const S *words = reinterpret_cast<const S *>(vals);
  auto value_at = [&](uint32_t d) -> S { return d < static_cast<uint32_t>(kRefreshWords) ? words[d] : S{}; };
  // Wave w takes panels w, w + 16, ... in batches of kRefreshPanels: the
  // word loads of all of a batch's segments are issued before the first is
  // used.  Segments start on a multiple of 4 entries, so dest + a is 8-byte
  // and out + a 4 * sizeof(S)-byte aligned.
  auto *oq = reinterpret_cast<RefreshQuad<S> *>(out);
  for (int64_t qb = 0; qb < n_panels; qb += kRefreshWaves * kRefreshPanels) {
    int64_t a[kRefreshPanels];
    uint32_t len4[kRefreshPanels], most = 0;
    __amdgpu_buffer_rsrc_t rd[kRefreshPanels];
#pragma unroll
    for (int k = 0; k < kRefreshPanels; ++k) {
      const int64_t q = qb + wave + static_cast<int64_t>(kRefreshWaves) * k;
      a[k] = q < n_panels ? static_cast<int64_t>(seg[q * n_tiles + t]) : 0;
      len4[k] = q < n_panels ? static_cast<uint32_t>(seg[q * n_tiles + t + 1] - a[k]) / 4u : 0u;
      most = len4[k] > most ? len4[k] : most;
      rd[k] = make_rsrc(dest + a[k], uint64_t{8} * len4[k]);
    }
    for (uint32_t e = lane; e < most; e += kWave) {
      uint64_t d[kRefreshPanels];
#pragma unroll
      for (int k = 0; k < kRefreshPanels; ++k) d[k] = BufLoad<8, kCacheStream>::load(rd[k], 8u * e);
#pragma unroll
      for (int k = 0; k < kRefreshPanels; ++k) {
        if (e < len4[k]) {
          RefreshQuad<S> qv;
#pragma unroll
          for (int u = 0; u < 4; ++u) qv.v[u] = value_at(static_cast<uint32_t>((d[k] >> (16 * u)) & 0xFFFFu));
          oq[a[k] / 4 + e] = qv;
        }
      }
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

// Exclusive prefix sum of n + 1 counts (the last one 0) into out; returns
// the total through *total (host).
msx_status exclusive_scan(Scratch &tmp, const uint32_t *in, uint32_t *out, int64_t n,
                          uint32_t *total, hipStream_t stream) {
  size_t bytes = 0;
  MSX_HIP_TRY(hipcub::DeviceScan::ExclusiveSum(nullptr, bytes, in, out, static_cast<int>(n + 1), stream));
  void *scratch = nullptr;
  if (!tmp.alloc(&scratch, bytes)) return no_memory();
  MSX_HIP_TRY(hipcub::DeviceScan::ExclusiveSum(scratch, bytes, in, out, static_cast<int>(n + 1), stream));
  MSX_HIP_TRY(hipMemcpyAsync(total, out + n, sizeof(uint32_t), hipMemcpyDeviceToHost, stream));
  MSX_HIP_TRY(hipStreamSynchronize(stream));
  return MSX_OK;
}

// The layout over nv virtual rows delimited by rowptr (RP = the index type
// when the virtual rows are the rows, uint32_t for the virtual-row starts).
template <class V, class I, class RP>
msx_status build_layout(msx_csr_plan *p, const typename V::Storage *data, const I *indices,
                        const RP *rowptr, int64_t nv, hipStream_t stream) {
  using S = typename V::Storage;
  using A = typename V::Acc;
  const int64_t nnz = p->nnz, W = p->block_nnz;
  const int64_t PW = kPanelBytes / static_cast<int64_t>(sizeof(A));
  const int64_t TW = kTileBytes / static_cast<int64_t>(sizeof(A));
  const int64_t H = TW - W;
  const int64_t P = (p->n_cols + PW - 1) / PW;
  const int64_t n = nv;
  Scratch tmp{{}, stream};

  // Tiles.
  uint32_t *flag = nullptr, *tid = nullptr;
  if (!tmp.alloc(&flag, sizeof(uint32_t) * (n + 1)) || !tmp.alloc(&tid, sizeof(uint32_t) * (n + 1)))
    return no_memory();
  hipLaunchKernelGGL((tile_flags<RP>), dim3(grid_for(n + 1)), dim3(kThreads), 0, stream, rowptr, n,
                     nnz, H, flag);
  MSX_HIP_TRY(hipGetLastError());
  uint32_t n_tiles_u = 0;
  MSX_TRY_STATUS(exclusive_scan(tmp, flag, tid, n, &n_tiles_u, stream));
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
  hipLaunchKernelGGL(tile_bounds, dim3(grid_for(n)), dim3(kThreads), 0, stream, n, flag, tid,
                     p->pn_tile_begin, p->pn_tile_end);
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
  hipLaunchKernelGGL((panel_keys<I, RP>), dim3(grid_for(n)), dim3(kThreads), 0, stream, indices,
                     rowptr, n, nnz, p->n_cols, PW, TW, static_cast<uint32_t>(n_tiles), flag, tid,
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

  // Pass-1 chunks: one workgroup per CU fits (its x panel fills the LDS),
  // so the grid is C = min(CUs, values / kMinChunk) chunks - never more, or
  // it spills into a second, nearly empty round - split at panel
  // boundaries: panel q gets floor(C * len / total) chunks, at least one,
  // and the chunks left over go to the largest remainders.  With more
  // non-empty panels than C, each gets one.
  const int64_t C = std::max<int64_t>(1, std::min<int64_t>(cus, n_values / kMinChunk));
  std::vector<int64_t> per(static_cast<size_t>(P), 0), rem(static_cast<size_t>(P), -1);
  int64_t given = 0;
  for (int64_t q = 0; q < P; ++q) {
    const int64_t len = static_cast<int64_t>(pb[q + 1]) - static_cast<int64_t>(pb[q]);
    if (len <= 0) continue;
    per[q] = std::max<int64_t>(1, C * len / n_values);
    rem[q] = C * len % n_values;
    given += per[q];
  }
  while (given < C) {
    int64_t best = -1;
    for (int64_t q = 0; q < P; ++q)
      if (rem[q] >= 0 && (best < 0 || rem[q] > rem[best])) best = q;
    if (best < 0) break;
    ++per[best];
    rem[best] = -1;
    ++given;
  }
  std::vector<int64_t> cbeg;
  std::vector<int32_t> cpan;
  for (int64_t q = 0; q < P; ++q) {
    const int64_t a = pb[q], b = pb[q + 1];
    if (b <= a) continue;
    const int64_t c = per[q];
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
  p->pn_vrows = nv;
  {  // the widest tile in virtual rows (sizes the value-gradient LDS)
    std::vector<int32_t> tb(static_cast<size_t>(n_tiles)), te(static_cast<size_t>(n_tiles));
    MSX_HIP_TRY(hipMemcpyAsync(tb.data(), p->pn_tile_begin, sizeof(int32_t) * n_tiles,
                               hipMemcpyDeviceToHost, stream));
    MSX_HIP_TRY(hipMemcpyAsync(te.data(), p->pn_tile_end, sizeof(int32_t) * n_tiles,
                               hipMemcpyDeviceToHost, stream));
    MSX_HIP_TRY(hipStreamSynchronize(stream));
    int64_t widest = 1;
    for (int64_t t = 0; t < n_tiles; ++t) widest = std::max<int64_t>(widest, int64_t{te[t]} - tb[t]);
    p->pn_tile_rows_max = std::min<int64_t>(widest, TW);
  }
  return prepare_spmv_panels(p);
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
  if (p->n_long == 0) return build_layout<V, I, I>(p, data, indices, indptr, n, stream);

  // Virtual rows: long rows cut into chunks of W values.
  uint32_t nv_u = 0;
  uint32_t *count = nullptr, *vbase = nullptr;
  {
    Scratch tmp{{}, stream};
    if (!tmp.alloc(&count, sizeof(uint32_t) * (n + 1)) || !tmp.alloc(&vbase, sizeof(uint32_t) * (n + 1)))
      return no_memory();
    hipLaunchKernelGGL((vrow_counts<I>), dim3(grid_for(n + 1)), dim3(kThreads), 0, stream, indptr, n,
                       nnz, W, count);
    MSX_HIP_TRY(hipGetLastError());
    MSX_TRY_STATUS(exclusive_scan(tmp, count, vbase, n, &nv_u, stream));
    const int64_t nv = nv_u;
    const size_t b_base = round256(sizeof(uint32_t) * (n + 1));
    const size_t b_start = round256(sizeof(uint32_t) * (nv + 1));
    const size_t b_slot = round256(sizeof(int32_t) * std::max<int64_t>(nv, 1));
    const size_t b_part = round256(sizeof(A) * std::max<int64_t>(nv, 1));
    char *vm = nullptr;
    if (hipMalloc(&vm, b_base + b_start + b_slot + b_part) != hipSuccess) {
      (void)hipGetLastError();
      return no_memory();
    }
    p->pn_vmeta = vm;
    p->pn_bytes += b_base + b_start + b_slot + b_part;
    p->pn_vbase = reinterpret_cast<uint32_t *>(vm);
    p->pn_vstart = reinterpret_cast<uint32_t *>(vm + b_base);
    p->pn_vslot = reinterpret_cast<int32_t *>(vm + b_base + b_start);
    p->pn_partial = vm + b_base + b_start + b_slot;
    MSX_HIP_TRY(hipMemcpyAsync(p->pn_vbase, vbase, sizeof(uint32_t) * (n + 1),
                               hipMemcpyDeviceToDevice, stream));
    hipLaunchKernelGGL((vrow_fill<I>), dim3(grid_for(n + 1)), dim3(kThreads), 0, stream, indptr, n,
                       nnz, W, p->pn_vbase, p->pn_vstart, p->pn_vslot);
    MSX_HIP_TRY(hipGetLastError());
  }
  return build_layout<V, I, uint32_t>(p, data, indices, p->pn_vstart, nv_u, stream);
}

template <class V, class I>
msx_status refresh_typed(msx_csr_plan *p, const void *data, hipStream_t stream) {
  using S = typename V::Storage;
  if (p->n_tiles == 0 || p->pn_values == 0) return MSX_OK;
  if (p->tile_words != kTileBytes / static_cast<int64_t>(sizeof(typename V::Acc)))
    return fail(MSX_EINVAL, "msx_csr_plan_refresh: unexpected tile size in the panel layout.");
  const size_t lds = static_cast<size_t>(refresh_lds_bytes(p->tile_words, sizeof(S)));
  if (p->pn_vstart != nullptr) {
    MSX_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void *>(&panel_refresh<S, uint32_t>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize,
                                    static_cast<int>(lds)));
    hipLaunchKernelGGL((panel_refresh<S, uint32_t>), dim3(static_cast<uint32_t>(p->n_tiles)),
                       dim3(kRefreshThreads), lds, stream, static_cast<const S *>(data), p->pn_vstart,
                       p->nnz, p->pn_tile_begin, p->pn_tile_end, p->pn_seg, p->n_panels,
                       p->n_tiles, p->pn_dest, static_cast<S *>(p->pn_data));
  } else {
    MSX_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void *>(&panel_refresh<S, I>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize,
                                    static_cast<int>(lds)));
    hipLaunchKernelGGL((panel_refresh<S, I>), dim3(static_cast<uint32_t>(p->n_tiles)),
                       dim3(kRefreshThreads), lds, stream, static_cast<const S *>(data),
                       static_cast<const I *>(p->indptr), p->nnz, p->pn_tile_begin, p->pn_tile_end,
                       p->pn_seg, p->n_panels, p->n_tiles, p->pn_dest,
                       static_cast<S *>(p->pn_data));
  }
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
  // Virtual rows (int32 tile bounds): the rows plus the extra chunks of
  // long rows.  Tiles: key windows of the word range.
  const int64_t nv_max = p->n_rows + p->nnz / long_chunk(p->block_nnz) + p->n_long;
  const int64_t tiles_max = (p->nnz + nv_max) / H + 2;
  if (nv_max >= (int64_t{1} << 31) - 1) return false;
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
