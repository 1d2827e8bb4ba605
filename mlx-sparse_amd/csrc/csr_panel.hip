// csr_panel.hip - two-pass SpMV over the column-panel copy of a bound plan.
//
// Why: with columns scattered over a large x (the 4M-row random matrix: one
// random 4-byte gather per value over 16.8 MB), a direct SpMV is bound by
// the L2 request rate, not by HBM.  Holding x in LDS turns the gather into
// an LDS read, but LDS holds only a 128 KB panel of x, so the values are
// processed panel by panel and the row sums need a second pass:
//
//   pass 1  (panel_products) one workgroup per chunk of one panel's values:
//           load the panel of x into LDS (widened to the accumulator type),
//           stream the chunk's values and panel columns, write each product
//           a * x[col] - rounded exactly as the reference rounds it before
//           adding - to the product buffer in the copy's order.  Pure
//           streaming: 1024 threads, four values per lane per load.
//   pass 2  (panel_rows) one workgroup per row tile: read the tile's
//           segment of every panel (all loads issued before the first use),
//           place each product at its LDS word (stored position inside the
//           tile), then sum each row from LDS left to right with the
//           reference's rule - rows of 1..4 values start from their first
//           product, longer rows from zero (reference:
//           src/sparse/csr_matvec/csr_matvec.cpp:79-114) - and store y.
//
// Short rows therefore equal the reference CPU kernel bit for bit, for every
// value type.  Long rows (more than W values) keep the plan's chunked path.
// The layout and its construction are described in csr_panel_build.hip.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "msx_device.h"
#include "msx_internal.h"

namespace msx {
namespace {

constexpr int kThreads = 1024;
constexpr int kUnroll = 4;
constexpr int kWavesPerGroup = kThreads / kWave;
// Panel runs one pass-2 wave gathers per batch (16 waves x 8 = 128 panels,
// the count of a 16.8 MB float32 x).
constexpr int kRunsPerWave = 8;
// Row bounds each pass-2 thread loads before the tile's products.
constexpr int kRowsAhead = 4;

__device__ inline int64_t clamp64(int64_t v, int64_t lo, int64_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

// Product of two accumulator-type values, rounded as the reference's CPU
// kernel rounds a*x (common.h:58-79 there: widened operands, one product).
__device__ inline float amul(float a, float b) { return a * b; }
__device__ inline c64 amul(c64 a, c64 b) { return vmul<C64>(a, b); }

template <class S>
struct alignas(4 * sizeof(S)) Four {
  S v[4];
};

// Streams read once per call (the copy's values, columns and LDS words, the
// product buffer in pass 2) use non-temporal loads (measured: pass 1 139 ->
// 111 us on the headline shape).  Product stores stay ordinary: streaming
// stores were slower.
template <int B>
struct NtWord;
template <>
struct NtWord<8> {
  using T = uint32_t __attribute__((ext_vector_type(2)));
};
template <>
struct NtWord<16> {
  using T = uint32_t __attribute__((ext_vector_type(4)));
};

template <class T>
__device__ inline T nt_load(const T *p) {
  static_assert(sizeof(T) == 8 || sizeof(T) == 16 || sizeof(T) == 32, "size");
  if constexpr (sizeof(T) == 32) {
    using W = NtWord<16>::T;
    const W *w = reinterpret_cast<const W *>(p);
    struct Pair {
      W a, b;
    } r{__builtin_nontemporal_load(w), __builtin_nontemporal_load(w + 1)};
    return __builtin_bit_cast(T, r);
  } else {
    using W = typename NtWord<sizeof(T)>::T;
    return __builtin_bit_cast(T, __builtin_nontemporal_load(reinterpret_cast<const W *>(p)));
  }
}

// Stage panel [c0, c0 + w) of x into LDS, widened: 16-byte loads, eight per
// thread issued before the first LDS store (the unaligned case and the tail
// element by element).
template <class V>
__device__ inline void stage_panel(typename V::Acc *xs, const typename V::Storage *__restrict__ x,
                                   int64_t c0, int w) {
  using S = typename V::Storage;
  constexpr int E = 16 / static_cast<int>(sizeof(S));
  constexpr int L = 8;
  const S *src = x + c0;
  int done = 0;
  if ((reinterpret_cast<uintptr_t>(src) & 15) == 0) {
    const int nv = w / E;
    const auto *s4 = reinterpret_cast<const uint4 *>(src);
    for (int v0 = 0; v0 < nv; v0 += L * kThreads) {
      uint4 t[L];
#pragma unroll
      for (int u = 0; u < L; ++u) {
        const int v = v0 + u * kThreads + static_cast<int>(threadIdx.x);
        if (v < nv) t[u] = s4[v];
      }
#pragma unroll
      for (int u = 0; u < L; ++u) {
        const int v = v0 + u * kThreads + static_cast<int>(threadIdx.x);
        if (v < nv) {
          struct Pack {
            S e[E];
          };
          const Pack pk = __builtin_bit_cast(Pack, t[u]);
#pragma unroll
          for (int k = 0; k < E; ++k) xs[v * E + k] = V::widen(pk.e[k]);
        }
      }
    }
    done = nv * E;
  }
  for (int i = done + static_cast<int>(threadIdx.x); i < w; i += kThreads) xs[i] = V::widen(src[i]);
}

// Issue the loads of `bytes` bytes at `src` straight into LDS at `lds`
// (buffer-to-LDS loads: lane l's 16 bytes land at 16 l of its wave's 1 KB;
// bytes past `bytes` read zero).  The caller waits for them.
__device__ inline void issue_panel_direct(unsigned char *lds, const void *src, uint32_t bytes) {
  const auto r = make_rsrc(src, bytes);
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint32_t lane = threadIdx.x % kWave;
  for (uint32_t u = wave; u * 1024u < bytes; u += kWavesPerGroup)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        r, (__attribute__((address_space(3))) void *)(lds + u * 1024u), 16, u * 1024u + 16u * lane,
        0, 0, 0);
}

// A store that is not read back soon (the value gradient).
template <class T>
__device__ inline void nt_store(T *p, T v) {
  if constexpr (sizeof(T) == 8) {
    using W = NtWord<8>::T;
    __builtin_nontemporal_store(__builtin_bit_cast(W, v), reinterpret_cast<W *>(p));
  } else {
    __builtin_nontemporal_store(v, p);
  }
}

// Pass 1.  Each workgroup owns one chunk of one panel and is the only one on
// its compute unit (the panel fills the LDS), so the time until its panel of
// x is staged is time its stream stands still: kPrefetch quads per lane of
// the chunk are loaded before the panel, and formed once it is there.  The
// rest streams in batches of U quads per lane.  Measured on the headline
// shape: 152 -> 142 us against one prefetched batch of four and a staging
// loop of single loads.
// XONLY: the entry's x value itself (widened), not the product; the copy's
// values are not read (the value gradient's gather of x).
constexpr int kPrefetch = 8;

template <class V, bool XONLY = false>
__global__ void __launch_bounds__(kThreads)
    panel_products(const typename V::Storage *__restrict__ data, const uint16_t *__restrict__ col,
                   const typename V::Storage *__restrict__ x, int64_t n_cols,
                   typename V::Acc *__restrict__ prod, const int64_t *__restrict__ chunk_begin,
                   const int32_t *__restrict__ chunk_panel, int64_t n_values, int PW) {
  using S = typename V::Storage;
  using A = typename V::Acc;
  extern __shared__ __align__(16) unsigned char lds_raw[];
  A *xs = reinterpret_cast<A *>(lds_raw);
  const int c = blockIdx.x;
  const int64_t q = chunk_panel[c];
  const int64_t b = clamp64(chunk_begin[c], 0, n_values);
  const int64_t e = clamp64(chunk_begin[c + 1], b, n_values);
  const int64_t c0 = q * PW;
  const int w = static_cast<int>(clamp64(n_cols - c0, 0, PW));
  int64_t a = (b + 3) & ~int64_t{3};
  if (a > e) a = e;
  const int64_t nq = (e - a) / 4;
  const auto *d4 = reinterpret_cast<const Four<S> *>(data + a);
  const auto *k4 = reinterpret_cast<const uint2 *>(col + a);
  auto *o4 = reinterpret_cast<Four<A> *>(prod + a);
  // A valid copy has col < w; the mask keeps a corrupted one inside LDS.
  const uint32_t mask = static_cast<uint32_t>(PW - 1);
  auto term = [&](S dv, uint32_t cw) -> A {
    if constexpr (XONLY) {
      (void)dv;
      return xs[cw & mask];
    } else {
      return amul(V::widen(dv), xs[cw & mask]);
    }
  };
  auto quad = [&](const Four<S> &dd, uint2 kk) {
    Four<A> o;
    o.v[0] = term(dd.v[0], kk.x);
    o.v[1] = term(dd.v[1], kk.x >> 16);
    o.v[2] = term(dd.v[2], kk.y);
    o.v[3] = term(dd.v[3], kk.y >> 16);
    return o;
  };
  const int64_t t0 = threadIdx.x;
  // x needs no widening (float32, complex64): the panel goes straight into
  // LDS by buffer-to-LDS loads, issued before the prefetch of the chunk
  // (lane l's 16 bytes land at 16 l of its wave's 1 KB; bytes past the
  // panel read zero), so no registers hold it and no LDS stores copy it.
  constexpr bool kDirect = sizeof(S) == sizeof(A);
  if constexpr (kDirect) issue_panel_direct(lds_raw, x + c0, static_cast<uint32_t>(w) * sizeof(S));
  Four<S> pd[kPrefetch] = {};
  uint2 pk[kPrefetch] = {};
  if constexpr (kDirect) {
    // Unconditional loads through descriptors over the chunk's quads (quads
    // past it read zero and are never stored): a load under a branch would
    // be waited on inside it, and with it the panel loads issued before.
    const auto r_d = make_rsrc(d4, static_cast<uint64_t>(nq) * sizeof(Four<S>));
    const auto r_k = make_rsrc(k4, static_cast<uint64_t>(nq) * sizeof(uint2));
#pragma unroll
    for (int u = 0; u < kPrefetch; ++u) {
      const auto qi = static_cast<uint32_t>(t0 + u * kThreads);
      if constexpr (!XONLY)
        pd[u] = __builtin_bit_cast(
            Four<S>, (BufLoad<sizeof(Four<S>), kCacheStream>::load(r_d, qi * sizeof(Four<S>))));
      pk[u] = __builtin_bit_cast(uint2, (BufLoad<8, kCacheStream>::load(r_k, qi * 8u)));
    }
    // The panel's loads were issued first and loads complete in order: wait
    // until no more than the prefetch's loads are outstanding.
    constexpr int kLoadsPerQuad = XONLY ? 1 : (sizeof(Four<S>) == 32 ? 3 : 2);
    constexpr int kAfter = kPrefetch * kLoadsPerQuad;
    static_assert(kAfter < 64, "vmcnt field");
    // s_waitcnt: vmcnt in bits 3:0 and 15:14, expcnt 6:4 and lgkmcnt 11:8 at
    // their maxima (not waited on)
    __builtin_amdgcn_s_waitcnt((kAfter & 15) | ((kAfter >> 4) << 14) | (7 << 4) | (15 << 8));
  } else {
#pragma unroll
    for (int u = 0; u < kPrefetch; ++u)
      if (t0 + u * kThreads < nq) {
        if constexpr (!XONLY) pd[u] = nt_load(d4 + t0 + u * kThreads);
        pk[u] = nt_load(k4 + t0 + u * kThreads);
      }
    stage_panel<V>(xs, x, c0, w);
  }
  __syncthreads();
  for (int64_t i = b + threadIdx.x; i < a; i += kThreads)
    prod[i] = term(XONLY ? S{} : data[i], col[i]);
#pragma unroll
  for (int u = 0; u < kPrefetch; ++u)
    if (t0 + u * kThreads < nq) o4[t0 + u * kThreads] = quad(pd[u], pk[u]);
  // x only: no values are loaded, so twice the column loads are kept in flight
  constexpr int U = XONLY ? 2 * kUnroll : kUnroll;
  int64_t qd = t0 + kPrefetch * kThreads;
  for (; qd + (U - 1) * kThreads < nq; qd += U * kThreads) {
    Four<S> d[U] = {};
    uint2 k[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if constexpr (!XONLY) d[u] = nt_load(d4 + qd + u * kThreads);
      k[u] = nt_load(k4 + qd + u * kThreads);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) o4[qd + u * kThreads] = quad(d[u], k[u]);
  }
  for (; qd < nq; qd += kThreads) {
    Four<S> dd = {};
    if constexpr (!XONLY) dd = d4[qd];
    o4[qd] = quad(dd, k4[qd]);
  }
  for (int64_t i = a + 4 * nq + threadIdx.x; i < e; i += kThreads)
    prod[i] = term(XONLY ? S{} : data[i], col[i]);
}

// Four products of a segment (16-byte aligned: segments are padded to
// multiples of 4 entries).
template <class A>
struct alignas(4 * sizeof(A)) ProdQuad {
  A v[4];
};

// NQ quads per lane per batch: a wave's share of a tile (TW / 16 words on
// average) usually takes one batch.
// Rows of a tile are virtual rows delimited by rowptr: the matrix's rows
// (RP = the index type, indptr) or, with LONG, short rows and chunks of
// long rows (RP = uint32_t, the plan's virtual-row starts); vslot then
// names each one's row, or -1 for a chunk, whose sum goes to partial.
template <class V, class RP, bool LONG>
__global__ void __launch_bounds__(kThreads)
    panel_rows(const typename V::Acc *__restrict__ prod, const uint16_t *__restrict__ dest,
               const uint32_t *__restrict__ seg, int64_t n_tiles, int P,
               const int32_t *__restrict__ tile_begin, const int32_t *__restrict__ tile_end,
               const RP *__restrict__ indptr, int64_t n_rows, int64_t nnz,
               typename V::Storage *__restrict__ y, int zero_fill,
               const int32_t *__restrict__ vslot, typename V::Acc *__restrict__ partial) {
  using A = typename V::Acc;
  constexpr int TW = 65536 / static_cast<int>(sizeof(A));
  constexpr int NQ = TW / kThreads / 4;
  extern __shared__ __align__(16) unsigned char lds_raw[];
  A *buf = reinterpret_cast<A *>(lds_raw);  // TW words
  const int64_t T = xcd_remap(blockIdx.x, gridDim.x);
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
  // The bounds of the thread's first kRowsAhead rows are loaded now; their
  // latency overlaps the product loads (tiles of short rows hold up to a
  // few thousand rows, and a bound loaded inside the sum loop would cost a
  // dependent round trip per row).
  const int64_t r0 = clamp64(tile_begin[T], 0, n_rows);
  const int64_t r1 = clamp64(tile_end[T], r0, n_rows);
  const int64_t b0 = clamp64(static_cast<int64_t>(indptr[r0]), 0, nnz);
  RP s_ahead[kRowsAhead], e_ahead[kRowsAhead];
  int32_t slot_ahead[kRowsAhead];
#pragma unroll
  for (int k = 0; k < kRowsAhead; ++k) {
    const int64_t r = r0 + threadIdx.x + static_cast<int64_t>(k) * kThreads;
    s_ahead[k] = 0;
    e_ahead[k] = 0;
    slot_ahead[k] = 0;
    if (r < r1) {
      s_ahead[k] = indptr[r];
      e_ahead[k] = indptr[r + 1];
      if constexpr (LONG) slot_ahead[k] = vslot[r];
    }
  }
  if (zero_fill) {
    for (int i = threadIdx.x; i < TW; i += kThreads) buf[i] = vzero<A>();
    __syncthreads();
  }

  // Wave w owns panels qb + w + 16k (k < kRunsPerWave) of each batch of
  // 16 * kRunsPerWave panels.  Their segments (q, T) are concatenated in
  // quads: the run starts and the prefix of their quad counts are
  // wave-uniform, so a lane finds the run of its quad j with
  // kRunsPerWave - 1 scalar compares and every load address is known before
  // the first load is issued.  Consecutive lanes read consecutive quads.
  const auto *pq = reinterpret_cast<const ProdQuad<A> *>(prod);
  for (int qb = 0; qb < P; qb += kWavesPerGroup * kRunsPerWave) {
    uint32_t st[kRunsPerWave], pre[kRunsPerWave + 1];
    pre[0] = 0;
#pragma unroll
    for (int k = 0; k < kRunsPerWave; ++k) {
      const int q = qb + wave + kWavesPerGroup * k;
      uint32_t s = 0, e = 0;
      if (q < P) {
        s = seg[static_cast<int64_t>(q) * n_tiles + T];
        e = seg[static_cast<int64_t>(q) * n_tiles + T + 1];
      }
      st[k] = s / 4;
      pre[k + 1] = pre[k] + (e > s ? (e - s) / 4 : 0u);
    }
    const uint32_t total = pre[kRunsPerWave];
    for (uint32_t j0 = 0; j0 < total; j0 += NQ * kWave) {
      ProdQuad<A> pv[NQ];
      uint2 dv[NQ];
#pragma unroll
      for (int u = 0; u < NQ; ++u) {
        const uint32_t j = j0 + u * kWave + lane;
        dv[u] = uint2{0xFFFFFFFFu, 0xFFFFFFFFu};
        if (j < total) {
          uint32_t base = st[0], p0 = 0;
#pragma unroll
          for (int k = 1; k < kRunsPerWave; ++k)
            if (j >= pre[k]) {
              base = st[k];
              p0 = pre[k];
            }
          const uint32_t quad = base + (j - p0);
          pv[u] = nt_load(pq + quad);
          dv[u] = nt_load(reinterpret_cast<const uint2 *>(dest) + quad);
        }
      }
#pragma unroll
      for (int u = 0; u < NQ; ++u) {
        const uint32_t d[4] = {dv[u].x & 0xFFFFu, dv[u].x >> 16, dv[u].y & 0xFFFFu, dv[u].y >> 16};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (d[e] < static_cast<uint32_t>(TW)) buf[d[e]] = pv[u].v[e];
      }
    }
  }
  __syncthreads();

  int k_row = 0;
  for (int64_t r = r0 + threadIdx.x; r < r1; r += kThreads, ++k_row) {
    int64_t s, e;
    int32_t slot = 0;
    if (k_row < kRowsAhead) {
      // a select over the prefetched rows (no dynamic register indexing)
      RP sa = s_ahead[0], ea = e_ahead[0];
      int32_t la = slot_ahead[0];
#pragma unroll
      for (int k = 1; k < kRowsAhead; ++k)
        if (k_row == k) {
          sa = s_ahead[k];
          ea = e_ahead[k];
          la = slot_ahead[k];
        }
      s = static_cast<int64_t>(sa);
      e = static_cast<int64_t>(ea);
      slot = la;
    } else {
      s = static_cast<int64_t>(indptr[r]);
      e = static_cast<int64_t>(indptr[r + 1]);
      if constexpr (LONG) slot = vslot[r];
    }
    if constexpr (!LONG) slot = static_cast<int32_t>(r);
    s = clamp64(s, 0, nnz);
    e = clamp64(e, s, nnz);
    const int64_t base = clamp64((s - b0) + (r - r0), 0, TW);
    const int len = static_cast<int>(std::min<int64_t>(e - s, TW - base));
    const A *v = buf + base;
    A acc = vzero<A>();
    int i = 0;
    // a chunk of a long row sums from zero, like the long row it belongs to
    if (len >= 1 && len <= 4 && slot >= 0) {
      acc = v[0];
      i = 1;
    }
    // stored order; eight LDS reads are issued before their adds
    for (; i + 8 <= len; i += 8) {
      A t[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) t[u] = v[i + u];
#pragma unroll
      for (int u = 0; u < 8; ++u) acc = vadd(acc, t[u]);
    }
    for (; i < len; ++i) acc = vadd(acc, v[i]);
    if (slot >= 0)
      y[slot] = V::narrow(acc);
    else
      partial[r] = acc;
  }
}

// Long rows of a virtual-row layout: one 256-thread workgroup per long row
// adds its chunk sums - each thread a strided share (four loads in flight),
// then a butterfly per wave and the four wave sums in order - so the
// result is the same on every call.
constexpr int kFixupThreads = 256;

template <class V>
__global__ void __launch_bounds__(kFixupThreads)
    panel_long_fixup(const typename V::Acc *__restrict__ partial, const uint32_t *__restrict__ vbase,
                     const int32_t *__restrict__ long_rows, int64_t n_rows,
                     typename V::Storage *__restrict__ y) {
  using A = typename V::Acc;
  __shared__ A wave_sum[kFixupThreads / kWave];
  const int64_t r = long_rows[blockIdx.x];
  if (r < 0 || r >= n_rows) return;  // uniform across the workgroup
  const int64_t a = vbase[r], b = vbase[r + 1];
  A acc = vzero<A>();
  int64_t k = a + threadIdx.x;
  for (; k + 3 * kFixupThreads < b; k += 4 * kFixupThreads) {
    A t[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) t[u] = partial[k + u * kFixupThreads];
#pragma unroll
    for (int u = 0; u < 4; ++u) acc = vadd(acc, t[u]);
  }
  for (; k < b; k += kFixupThreads) acc = vadd(acc, partial[k]);
#pragma unroll
  for (int d = kWave / 2; d >= 1; d >>= 1) acc = vadd(acc, shfl_xor(acc, d));
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  if (lane == 0) wave_sum[wave] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    A total = wave_sum[0];
    for (int w = 1; w < kFixupThreads / kWave; ++w) total = vadd(total, wave_sum[w]);
    y[r] = V::narrow(total);
  }
}

// Value gradient of y = A x over the panel layout (out[p] = cot[row(p)] *
// x[col(p)], the same rounding as the plan-free kernel): the first pass is
// panel_products<V, true>, which writes each entry's x value; this second
// pass takes one workgroup per tile, like pass 2 of the SpMV.  In a tile's
// LDS words, virtual row v0 + i holds its values at words (p - b0) + i and
// one more word right after them, its gap.  Each row stores its cotangent
// in its gap and sets the gap's bit in a bitmap; each entry's x value goes
// to its word (the segment runs read as in pass 2).  Then the tile's words
// are walked in order, 64 per wave step - one bitmap word per step: a
// value word w's row i is the number of gaps before it (a prefix count per
// bitmap word plus a popcount), its cotangent sits in the next gap, and
// its gradient goes to position b0 + w - i, so the stores stay coalesced.
// A row whose gap lies past its bitmap word takes the first gap of a later
// word, precomputed per word (a suffix minimum) so that no lane searches.
// LDS: the words, TW / 8 bytes of bitmap, a count and a next gap per bitmap
// word (68 KB for 4-byte accumulators), so two workgroups share a compute
// unit.  Only for copies that dropped no value (every value word is then
// written).
template <class V, class RP, bool LONG>
__global__ void __launch_bounds__(kThreads)
    panel_vjp_scatter(const typename V::Acc *__restrict__ xg, const uint16_t *__restrict__ dest,
                      const uint32_t *__restrict__ seg, int64_t n_tiles, int P,
                      const int32_t *__restrict__ tile_begin, const int32_t *__restrict__ tile_end,
                      const RP *__restrict__ rowptr, const int32_t *__restrict__ vslot, int64_t nv,
                      int64_t nnz, int rows_cap, const typename V::Storage *__restrict__ cot,
                      typename V::Storage *__restrict__ out) {
  using A = typename V::Acc;
  constexpr int TW = 65536 / static_cast<int>(sizeof(A));
  constexpr int NQ = TW / kThreads / 4;
  constexpr int NB = TW / 64;  // bitmap words
  static_assert(NB <= kThreads, "one thread per bitmap word");
  extern __shared__ __align__(16) unsigned char lds_raw[];
  A *xw = reinterpret_cast<A *>(lds_raw);                                        // TW words
  unsigned long long *gap = reinterpret_cast<unsigned long long *>(xw + TW);     // NB
  uint32_t *before = reinterpret_cast<uint32_t *>(gap + NB);                     // NB
  uint32_t *wsum = before + NB;                                                  // one per wave
  int32_t *nextg = reinterpret_cast<int32_t *>(wsum + kWavesPerGroup);           // NB
  int32_t *wmin = nextg + NB;                                                    // one per wave
  const int64_t T = xcd_remap(blockIdx.x, gridDim.x);
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
  const int64_t v0 = clamp64(tile_begin[T], 0, nv);
  const int64_t v1 = clamp64(tile_end[T], v0, std::min<int64_t>(nv, v0 + rows_cap));
  const int64_t b0 = clamp64(static_cast<int64_t>(rowptr[v0]), 0, nnz);
  const int64_t b1 = clamp64(static_cast<int64_t>(rowptr[v1]), b0, std::min<int64_t>(nnz, b0 + TW));
  if (threadIdx.x < NB) gap[threadIdx.x] = 0;
  // The bounds (and, for rows that are their own virtual row, the
  // cotangents) of the thread's first kRowsAhead rows are loaded before the
  // tile's x values, so that their latency overlaps those loads; they go to
  // LDS after the runs.
  int64_t s_ahead[kRowsAhead], e_ahead[kRowsAhead];
  A c_ahead[kRowsAhead];
  int32_t slot_ahead[kRowsAhead];
#pragma unroll
  for (int k = 0; k < kRowsAhead; ++k) {
    const int64_t v = v0 + threadIdx.x + static_cast<int64_t>(k) * kThreads;
    s_ahead[k] = 0;
    e_ahead[k] = 0;
    c_ahead[k] = vzero<A>();
    slot_ahead[k] = 0;
    if (v < v1) {
      s_ahead[k] = static_cast<int64_t>(rowptr[v]);
      e_ahead[k] = static_cast<int64_t>(rowptr[v + 1]);
      if constexpr (LONG)
        slot_ahead[k] = vslot[v];
      else
        c_ahead[k] = V::widen(cot[v]);
    }
  }
  __syncthreads();  // the bitmap is clear

  const auto *xq = reinterpret_cast<const ProdQuad<A> *>(xg);
  for (int qb = 0; qb < P; qb += kWavesPerGroup * kRunsPerWave) {
    uint32_t st[kRunsPerWave], pre[kRunsPerWave + 1];
    pre[0] = 0;
#pragma unroll
    for (int k = 0; k < kRunsPerWave; ++k) {
      const int q = qb + wave + kWavesPerGroup * k;
      uint32_t s = 0, e = 0;
      if (q < P) {
        s = seg[static_cast<int64_t>(q) * n_tiles + T];
        e = seg[static_cast<int64_t>(q) * n_tiles + T + 1];
      }
      st[k] = s / 4;
      pre[k + 1] = pre[k] + (e > s ? (e - s) / 4 : 0u);
    }
    const uint32_t total = pre[kRunsPerWave];
    for (uint32_t j0 = 0; j0 < total; j0 += NQ * kWave) {
      ProdQuad<A> xv[NQ];
      uint2 dv[NQ];
#pragma unroll
      for (int u = 0; u < NQ; ++u) {
        const uint32_t j = j0 + u * kWave + lane;
        dv[u] = uint2{0xFFFFFFFFu, 0xFFFFFFFFu};
        if (j < total) {
          uint32_t base = st[0], p0 = 0;
#pragma unroll
          for (int k = 1; k < kRunsPerWave; ++k)
            if (j >= pre[k]) {
              base = st[k];
              p0 = pre[k];
            }
          const uint32_t quad = base + (j - p0);
          xv[u] = nt_load(xq + quad);
          dv[u] = nt_load(reinterpret_cast<const uint2 *>(dest) + quad);
        }
      }
#pragma unroll
      for (int u = 0; u < NQ; ++u) {
        const uint32_t d[4] = {dv[u].x & 0xFFFFu, dv[u].x >> 16, dv[u].y & 0xFFFFu, dv[u].y >> 16};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (d[e] < static_cast<uint32_t>(TW)) xw[d[e]] = xv[u].v[e];
      }
    }
  }

  // Rows: the cotangent into the gap word, the gap's bit into the bitmap.
  int k_row = 0;
  for (int64_t v = v0 + threadIdx.x; v < v1; v += kThreads, ++k_row) {
    int64_t s, e;
    A c;
    if (k_row < kRowsAhead) {
      // a select over the prefetched rows (no dynamic register indexing)
      s = s_ahead[0];
      e = e_ahead[0];
      c = c_ahead[0];
      int32_t slot = slot_ahead[0];
#pragma unroll
      for (int k = 1; k < kRowsAhead; ++k)
        if (k_row == k) {
          s = s_ahead[k];
          e = e_ahead[k];
          c = c_ahead[k];
          slot = slot_ahead[k];
        }
      if constexpr (LONG) c = V::widen(cot[slot >= 0 ? slot : -1 - static_cast<int64_t>(slot)]);
    } else {
      s = static_cast<int64_t>(rowptr[v]);
      e = static_cast<int64_t>(rowptr[v + 1]);
      int64_t r = v;
      if constexpr (LONG) {
        const int32_t slot = vslot[v];
        r = slot >= 0 ? slot : -1 - static_cast<int64_t>(slot);
      }
      c = V::widen(cot[r]);
    }
    s = clamp64(s, b0, b1);
    e = clamp64(e, s, b1);
    const int64_t g = (e - b0) + (v - v0);
    if (g < TW) {
      xw[g] = c;
      atomicOr(&gap[g >> 6], 1ull << (g & 63));
    }
  }
  __syncthreads();

  // Gaps before each bitmap word: a scan of the NB counts (a wave scan,
  // then the wave totals in order).
  {
    uint32_t c = threadIdx.x < NB ? static_cast<uint32_t>(__popcll(gap[threadIdx.x])) : 0u;
    uint32_t incl = c;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const uint32_t t = __shfl_up(incl, d, kWave);
      if (lane >= d) incl += t;
    }
    if (lane == kWave - 1) wsum[wave] = incl;
    __syncthreads();
    uint32_t off = 0;
    for (int w = 0; w < wave; ++w) off += wsum[w];
    if (threadIdx.x < NB) before[threadIdx.x] = off + incl - c;
    // The first gap after each bitmap word (where the last row that starts
    // in the word has its gap when it runs past the word): an exclusive
    // suffix minimum of the words' first gaps.
    int32_t first = INT32_MAX;
    if (threadIdx.x < NB) {
      const unsigned long long b = gap[threadIdx.x];
      if (b != 0) first = static_cast<int32_t>(threadIdx.x) * 64 + static_cast<int32_t>(__builtin_ctzll(b));
    }
    int32_t suf = first;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const int32_t t = __shfl_down(suf, d, kWave);
      if (lane + d < kWave) suf = t < suf ? t : suf;
    }
    if (lane == 0) wmin[wave] = suf;
    __syncthreads();
    int32_t later = INT32_MAX;
    for (int v = wave + 1; v < NB / kWave; ++v) later = wmin[v] < later ? wmin[v] : later;
    int32_t next_in_wave = __shfl_down(suf, 1, kWave);
    if (lane == kWave - 1) next_in_wave = INT32_MAX;
    if (threadIdx.x < NB) nextg[threadIdx.x] = next_in_wave < later ? next_in_wave : later;
    __syncthreads();
  }

  // The walk: thread t holds the WPT consecutive words from t * WPT, all in
  // one bitmap word.  The cotangent of a value word is the word of the next
  // gap: inside the chunk, found going backwards over its words; after the
  // chunk's last gap, the first gap above the chunk (in this bitmap word, or
  // a later one's first gap).  A value word's position is its word minus the
  // gaps below it, so the chunk's products land at consecutive positions;
  // they are written over the words (after every chunk has been read) and
  // then stored from LDS in position order, coalesced.
  constexpr int WPT = TW / kThreads;  // 16 words (4-byte accumulators), 8 (complex64)
  static_assert(WPT * kThreads == TW && 64 % WPT == 0, "a chunk lies in one bitmap word");
  const uint32_t npos = static_cast<uint32_t>(b1 - b0);
  const int w0 = static_cast<int>(threadIdx.x) * WPT;
  const int k = w0 >> 6, sh = w0 & 63;
  const unsigned long long bits = gap[k];
  const uint32_t cbits = static_cast<uint32_t>((bits >> sh) & ((1ull << WPT) - 1ull));
  // gaps below the chunk
  const uint32_t gb = before[k] + static_cast<uint32_t>(__popcll(bits & ((1ull << sh) - 1ull)));
  const unsigned long long above = sh + WPT < 64 ? bits >> (sh + WPT) : 0ull;
  const int later = nextg[k];
  const int tail_g = above != 0 ? w0 + WPT + static_cast<int>(__builtin_ctzll(above)) : later;
  using Chunk = Four<A>;  // four words per LDS read
  Chunk cv[WPT / 4];
#pragma unroll
  for (int u = 0; u < WPT / 4; ++u) cv[u] = reinterpret_cast<const Chunk *>(xw + w0)[u];
  // (no gap above the chunk: its words after its last gap lie past the
  // tile's last row, at positions >= npos, which are not written)
  A c = xw[tail_g < TW ? tail_g : 0];
  __syncthreads();  // every chunk and tail read before the products overwrite the words
  A prod[WPT];
#pragma unroll
  for (int i = WPT - 1; i >= 0; --i) {
    const A v = cv[i / 4].v[i % 4];
    prod[i] = amul(c, v);
    if ((cbits >> i) & 1u) c = v;
  }
  uint32_t pos = static_cast<uint32_t>(w0) - gb;
#pragma unroll
  for (int i = 0; i < WPT; ++i) {
    if (!((cbits >> i) & 1u)) {
      if (pos < npos) xw[pos] = prod[i];
      ++pos;
    }
  }
  __syncthreads();
  typename V::Storage *ob = out + b0;
#pragma unroll 4
  for (uint32_t q = threadIdx.x; q < npos; q += kThreads) nt_store(ob + q, V::narrow(xw[q]));
}

template <class A>
size_t pass1_lds(const msx_csr_plan *p) {
  return sizeof(A) * static_cast<size_t>(p->panel_width);
}

template <class A>
size_t pass2_lds(const msx_csr_plan *p) {
  return sizeof(A) * static_cast<size_t>(p->tile_words);
}

// LDS of one workgroup on gfx950.
constexpr size_t kMaxLdsBytes = 163840;

// Value-gradient pass 2: the words (x values and gap cotangents), the gap
// bitmap, the gaps before each bitmap word, one count per wave.
template <class A>
size_t vjp_lds(const msx_csr_plan *p) {
  const size_t words = static_cast<size_t>(p->tile_words);
  return sizeof(A) * words + (words / 64) * (sizeof(unsigned long long) + 2 * sizeof(uint32_t)) +
         2 * sizeof(uint32_t) * kWavesPerGroup;
}

// Both passes take more than 64 KB of dynamic LDS.  The limit is raised
// when a plan is built (on the plan's device), never inside a launch, so a
// launch stays legal under stream capture.
template <class V, class I>
msx_status prepare_typed(const msx_csr_plan *p) {
  using A = typename V::Acc;
  MSX_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void *>(&panel_products<V>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize,
                                  static_cast<int>(pass1_lds<A>(p))));
  MSX_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void *>(&panel_rows<V, I, false>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize,
                                  static_cast<int>(pass2_lds<A>(p))));
  MSX_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void *>(&panel_rows<V, uint32_t, true>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize,
                                  static_cast<int>(pass2_lds<A>(p))));
  MSX_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void *>(&panel_products<V, true>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize,
                                  static_cast<int>(pass1_lds<A>(p))));
  if (vjp_lds<A>(p) <= kMaxLdsBytes) {
    MSX_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void *>(&panel_vjp_scatter<V, I, false>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize,
                                    static_cast<int>(vjp_lds<A>(p))));
    MSX_HIP_TRY(hipFuncSetAttribute(
        reinterpret_cast<const void *>(&panel_vjp_scatter<V, uint32_t, true>),
        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(vjp_lds<A>(p))));
  }
  return MSX_OK;
}

template <class V>
msx_status prepare_v(const msx_csr_plan *p) {
  return p->itype == MSX_I32 ? prepare_typed<V, int32_t>(p) : prepare_typed<V, int64_t>(p);
}

template <class V, class I>
msx_status launch_typed(const msx_csr_plan *p, const void *indptr, const void *x, void *y,
                        hipStream_t stream) {
  using S = typename V::Storage;
  using A = typename V::Acc;
  const size_t lds1 = pass1_lds<A>(p);
  hipLaunchKernelGGL((panel_products<V>), dim3(static_cast<uint32_t>(p->pn_chunks)), dim3(kThreads), lds1,
                     stream, static_cast<const S *>(p->pn_data), p->pn_col, static_cast<const S *>(x),
                     p->n_cols, static_cast<A *>(p->pn_prod), p->pn_chunk_begin, p->pn_chunk_panel,
                     p->pn_values, static_cast<int>(p->panel_width));
  MSX_HIP_TRY(hipGetLastError());
  const size_t lds2 = pass2_lds<A>(p);
  if (p->pn_vstart == nullptr) {
    hipLaunchKernelGGL((panel_rows<V, I, false>), dim3(static_cast<uint32_t>(p->n_tiles)),
                       dim3(kThreads), lds2, stream, static_cast<const A *>(p->pn_prod), p->pn_dest,
                       p->pn_seg, p->n_tiles, static_cast<int>(p->n_panels), p->pn_tile_begin,
                       p->pn_tile_end, static_cast<const I *>(indptr), p->n_rows, p->nnz,
                       static_cast<S *>(y), p->pn_dropped ? 1 : 0, nullptr, nullptr);
    MSX_HIP_TRY(hipGetLastError());
    return MSX_OK;
  }
  // Long rows: pass 2 writes their chunk sums, the fixup adds them.
  hipLaunchKernelGGL((panel_rows<V, uint32_t, true>), dim3(static_cast<uint32_t>(p->n_tiles)),
                     dim3(kThreads), lds2, stream, static_cast<const A *>(p->pn_prod), p->pn_dest,
                     p->pn_seg, p->n_tiles, static_cast<int>(p->n_panels), p->pn_tile_begin,
                     p->pn_tile_end, p->pn_vstart, p->pn_vrows, p->nnz, static_cast<S *>(y),
                     p->pn_dropped ? 1 : 0, p->pn_vslot, static_cast<A *>(p->pn_partial));
  MSX_HIP_TRY(hipGetLastError());
  hipLaunchKernelGGL((panel_long_fixup<V>), dim3(static_cast<uint32_t>(p->n_long)),
                     dim3(kFixupThreads), 0, stream, static_cast<const A *>(p->pn_partial), p->pn_vbase,
                     p->long_rows, p->n_rows, static_cast<S *>(y));
  MSX_HIP_TRY(hipGetLastError());
  return MSX_OK;
}

template <class V, class I>
msx_status vjp_typed(const msx_csr_plan *p, const void *indptr, const void *x, const void *cot,
                     void *out, hipStream_t stream) {
  using S = typename V::Storage;
  using A = typename V::Acc;
  hipLaunchKernelGGL((panel_products<V, true>), dim3(static_cast<uint32_t>(p->pn_chunks)),
                     dim3(kThreads), pass1_lds<A>(p), stream, static_cast<const S *>(p->pn_data), p->pn_col,
                     static_cast<const S *>(x), p->n_cols, static_cast<A *>(p->pn_prod),
                     p->pn_chunk_begin, p->pn_chunk_panel, p->pn_values,
                     static_cast<int>(p->panel_width));
  MSX_HIP_TRY(hipGetLastError());
  const size_t lds = vjp_lds<A>(p);
  const int cap = static_cast<int>(p->pn_tile_rows_max);
  if (p->pn_vstart == nullptr)
    hipLaunchKernelGGL((panel_vjp_scatter<V, I, false>), dim3(static_cast<uint32_t>(p->n_tiles)),
                       dim3(kThreads), lds, stream, static_cast<const A *>(p->pn_prod), p->pn_dest,
                       p->pn_seg, p->n_tiles, static_cast<int>(p->n_panels), p->pn_tile_begin,
                       p->pn_tile_end, static_cast<const I *>(indptr), nullptr, p->n_rows, p->nnz,
                       cap, static_cast<const S *>(cot), static_cast<S *>(out));
  else
    hipLaunchKernelGGL((panel_vjp_scatter<V, uint32_t, true>), dim3(static_cast<uint32_t>(p->n_tiles)),
                       dim3(kThreads), lds, stream, static_cast<const A *>(p->pn_prod), p->pn_dest,
                       p->pn_seg, p->n_tiles, static_cast<int>(p->n_panels), p->pn_tile_begin,
                       p->pn_tile_end, p->pn_vstart, p->pn_vslot, p->pn_vrows, p->nnz, cap,
                       static_cast<const S *>(cot), static_cast<S *>(out));
  MSX_HIP_TRY(hipGetLastError());
  return MSX_OK;
}

template <class V>
msx_status launch_v(const msx_csr_plan *p, const void *indptr, const void *x, void *y,
                    hipStream_t stream) {
  return p->itype == MSX_I32 ? launch_typed<V, int32_t>(p, indptr, x, y, stream)
                             : launch_typed<V, int64_t>(p, indptr, x, y, stream);
}

}  // namespace

msx_status prepare_spmv_panels(const msx_csr_plan *p) {
  switch (p->vtype) {
  case MSX_F32: return prepare_v<F32>(p);
  case MSX_F16: return prepare_v<F16>(p);
  case MSX_BF16: return prepare_v<BF16>(p);
  case MSX_C64: return prepare_v<C64>(p);
  }
  return fail(MSX_ETYPE, "msx_csr_plan_create_bound unsupported value dtype.");
}

bool panel_data_vjp_fits(const msx_csr_plan *p) {
  if (p->n_panels == 0 || p->pn_dropped) return false;
  return (p->vtype == MSX_C64 ? vjp_lds<c64>(p) : vjp_lds<float>(p)) <= kMaxLdsBytes;
}

msx_status launch_panel_data_vjp(const msx_csr_plan *p, const void *indptr, const void *x,
                                 const void *cot, void *out, hipStream_t stream) {
  const bool i32 = p->itype == MSX_I32;
  switch (p->vtype) {
  case MSX_F32: return i32 ? vjp_typed<F32, int32_t>(p, indptr, x, cot, out, stream)
                           : vjp_typed<F32, int64_t>(p, indptr, x, cot, out, stream);
  case MSX_F16: return i32 ? vjp_typed<F16, int32_t>(p, indptr, x, cot, out, stream)
                           : vjp_typed<F16, int64_t>(p, indptr, x, cot, out, stream);
  case MSX_BF16: return i32 ? vjp_typed<BF16, int32_t>(p, indptr, x, cot, out, stream)
                            : vjp_typed<BF16, int64_t>(p, indptr, x, cot, out, stream);
  case MSX_C64: return i32 ? vjp_typed<C64, int32_t>(p, indptr, x, cot, out, stream)
                           : vjp_typed<C64, int64_t>(p, indptr, x, cot, out, stream);
  }
  return fail(MSX_ETYPE, "csr_matvec_data_vjp unsupported value dtype.");
}

msx_status launch_spmv_panels(const msx_csr_plan *p, const void *indptr, const void *x, void *y,
                              hipStream_t stream) {
  switch (p->vtype) {
  case MSX_F32: return launch_v<F32>(p, indptr, x, y, stream);
  case MSX_F16: return launch_v<F16>(p, indptr, x, y, stream);
  case MSX_BF16: return launch_v<BF16>(p, indptr, x, y, stream);
  case MSX_C64: return launch_v<C64>(p, indptr, x, y, stream);
  }
  return fail(MSX_ETYPE, "msx_csr_spmv unsupported value dtype.");
}

}  // namespace msx
