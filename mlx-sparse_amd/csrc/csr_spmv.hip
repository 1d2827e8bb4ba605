// csr_spmv.hip - CSR SpMV kernels for gfx950.
//
//   y[i] = sum_{p in [indptr[i], indptr[i+1])} data[p] * x[indices[p]]
//
// The reference computes this with one Metal thread per row, or a 128-lane
// threadgroup per row when nnz >= 32 * n_rows, each lane reading data/indices
// strided by the row length (reference:
// src/sparse/csr_matvec/csr_matvec.metal:17-36,76-108).  Here the work comes
// from a row-block plan (csr_plan.hip):
//
//   spmv_blocks      one wavefront per short block (< 2W values, <= R rows).
//                    Phase 1 streams the block's contiguous indices/data with
//                    8-32 byte buffer loads (4 values per lane per load; the
//                    buffer descriptor returns zero past the array end, so the
//                    ragged edges need no scalar tail), gathers x, and stages
//                    the products in LDS.  Phase 2 sums each row from LDS:
//                    one lane per row in stored order when rows average <= 32
//                    values (the reference's summation order, so results
//                    match its CPU kernel bit for bit), otherwise L lanes per
//                    row and an XOR butterfly.
//   spmv_long        one 256-thread workgroup per C-value chunk of a long
//                    row; a fixed-order tree gives each chunk's sum.
//   spmv_long_fixup  one wavefront per multi-chunk row adds the chunk sums.
//   spmv_rowgroup    plan-free kernel: G lanes per row, G from the mean row
//                    length.  Used without a plan or for misaligned buffers.
//
// Every x gather is guarded by 0 <= col < n_cols (an out-of-range column
// adds nothing), and row bounds are clamped to [0, nnz], so malformed CSR
// input cannot read outside the caller's buffers.  No atomics: repeated
// calls produce identical bits.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "msx_device.h"
#include "msx_internal.h"
#include "msx_long_slice.h"

namespace msx {
namespace {

#define MSX_HIP_TRY_ST(expr)         \
  do {                               \
    msx_status _s = (expr);          \
    if (_s != MSX_OK) return _s;     \
  } while (0)

constexpr int kThreads = 256;
constexpr int kWavesPerGroup = kThreads / kWave;
constexpr uint32_t kMaxGrid = 1u << 20;  // workgroups per launch; kernels stride beyond

__device__ inline int64_t clamp64(int64_t v, int64_t lo, int64_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

// Offset from a0 of a row pointer clamped into its block [p0, p1].  With
// int32 row pointers p0, p1 and a0 are row-pointer values too, so the clamp
// runs in 32 bits.
__device__ inline int32_t block_offset(int32_t v, int64_t p0, int64_t p1, int64_t a0) {
  return std::min(std::max(v, static_cast<int32_t>(p0)), static_cast<int32_t>(p1)) -
         static_cast<int32_t>(a0);
}
__device__ inline int32_t block_offset(int64_t v, int64_t p0, int64_t p1, int64_t a0) {
  return static_cast<int32_t>(clamp64(v, p0, p1) - a0);
}

__device__ inline void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// --------------------------------------------------------------------------
// Short blocks.  W is a compile-time constant so each lane holds its whole
// share of the block (QPL quads of 4 values) in registers: all index/value
// loads of the block are issued before the first x gather, and all gathers
// before the first use, so a wave keeps ~8 loads and 4*QPL gathers in flight
// per lane.  The dependent chain per block is: plan entries -> (row pointers,
// indices, values) -> x gathers -> LDS -> y.
constexpr int kBlockRows = 256;  // R; equals the plan's block_rows

// Phase 1 of a short block, NC chunks of 64 quads (4 values per lane per
// load): all index/value quads, then all gathers, then the products staged
// in LDS.  The loads are unconditional - the descriptors end at p1, so
// quads past the block read zero - which lets the compiler issue every one
// before it waits on any; a load under a branch would be waited on inside
// it.  Products are staged for every loaded position: phase 2 reads only the
// row ranges, which lie inside the block.
template <class V, class I, int W, int AUX, int NC>
__device__ __forceinline__ void block_products(const typename V::Storage *__restrict__ data,
                                               const I *__restrict__ indices,
                                               const typename V::Storage *__restrict__ x,
                                               int64_t a0, int64_t p1, int64_t n_cols,
                                               uint32_t lim32, uint32_t x_bytes, int lane,
                                               typename V::Acc *prod) {
  using S = typename V::Storage;
  using A = typename V::Acc;
  constexpr int kQuads = W / 2 + 1;
  const auto ri = make_rsrc(indices + a0, static_cast<uint64_t>(p1 - a0) * sizeof(I));
  const auto rd = make_rsrc(data + a0, static_cast<uint64_t>(p1 - a0) * sizeof(S));
  Quad<I> iq[NC];
  Quad<S> dq[NC];
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    const uint32_t q = static_cast<uint32_t>(lane + k * kWave);
    iq[k] = load_quad<I, AUX>(ri, q * 4u * sizeof(I));
    dq[k] = load_quad<S, AUX>(rd, q * 4u * sizeof(S));
  }
  A xv[NC][4];
  if (x_bytes != 0) {
    const auto rx = make_rsrc(x, x_bytes);
    GatherRaw<S> raw[NC][4];
#pragma unroll
    for (int k = 0; k < NC; ++k)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        raw[k][e] = gather_raw<S>(rx, x_bytes, static_cast<uint32_t>(iq[k].v[e]),
                                  col_ok(iq[k].v[e], n_cols, lim32));
    // every gather is issued before the first is used
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < NC; ++k)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        xv[k][e] = gather_widen<V>(raw[k][e], static_cast<uint32_t>(iq[k].v[e]));
  } else {  // x beyond a descriptor's reach: clamped global loads
#pragma unroll
    for (int k = 0; k < NC; ++k) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const I col = iq[k].v[e];
        const bool ok = col_ok(col, n_cols, lim32);
        A v = vzero<A>();
        if (n_cols > 0) v = V::widen(x[ok ? static_cast<int64_t>(col) : 0]);  // wave-uniform test
        xv[k][e] = v;
      }
    }
  }
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    const int q = lane + k * kWave;
    if (W >= 128 || q < kQuads) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const A pv = vmul_acc<V>(xv[k][e], dq[k].v[e]);
        prod[4 * q + e] = col_ok(iq[k].v[e], n_cols, lim32) ? pv : vzero<A>();
      }
    }
  }
}

// block_products for the block's chunk count nch <= NC (a wave-uniform
// dispatch, so each case is straight-line code).
template <class V, class I, int W, int AUX, int NC>
__device__ __forceinline__ void block_products_n(int nch,
                                                 const typename V::Storage *__restrict__ data,
                                                 const I *__restrict__ indices,
                                                 const typename V::Storage *__restrict__ x,
                                                 int64_t a0, int64_t p1, int64_t n_cols,
                                                 uint32_t lim32, uint32_t x_bytes, int lane,
                                                 typename V::Acc *prod) {
  if constexpr (NC > 0) {
    if (nch >= NC)
      block_products<V, I, W, AUX, NC>(data, indices, x, a0, p1, n_cols, lim32, x_bytes, lane,
                                       prod);
    else
      block_products_n<V, I, W, AUX, NC - 1>(nch, data, indices, x, a0, p1, n_cols, lim32,
                                             x_bytes, lane, prod);
  }
}

// FUSE: the XCD-sliced long-row pieces ride in the same launch.  The first
// `long_groups` workgroups (a multiple of 8, so workgroup g still runs on
// XCD g % 8) sum long-row pieces, the rest walk the short blocks; the two
// halves gather from different places (one slice of x per XCD, all of x),
// so they overlap instead of running back to back.
// 16-bit values with int32 indices at W = 512, and complex64 with int32
// indices at W = 256 outside the fused launch, are held to 72 registers, 7
// waves per SIMD instead of 6 (banded f16 / bf16: 71 -> 67 us, complex64
// 128 -> 123 us; float32 runs slower so, 75 -> 78 us, and keeps its 78
// registers; the other variants would spill).
template <class V, class I, int W, int AUX, bool FUSE>
__global__ void __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu((W == 512 && sizeof(I) == 4 && sizeof(typename V::Storage) == 2) ||
                                    (W == 256 && !FUSE && sizeof(I) == 4 && sizeof(typename V::Storage) == 8)
                                ? 7
                                : 1,
                                8)))
    spmv_blocks(const typename V::Storage *__restrict__ data, const I *__restrict__ indices,
                const I *__restrict__ indptr, const typename V::Storage *__restrict__ x,
                typename V::Storage *__restrict__ y, const int32_t *__restrict__ bounds,
                const int64_t *__restrict__ bounds_nnz, int64_t n_bounds, int64_t nnz,
                int64_t n_cols, uint32_t x_bytes, uint32_t long_groups,
                const int64_t *__restrict__ ls_begin, const int32_t *__restrict__ ls_len,
                const int32_t *__restrict__ ls_slot, const int32_t *__restrict__ ls_slice_begin,
                typename V::Acc *__restrict__ ls_partial) {
  // FUSE: workgroups come in octets (workgroup g runs on XCD g % 8); the
  // long_groups / 8 long-piece octets are spread evenly through the grid,
  // so both kinds of work run side by side for the whole launch.
  uint32_t gid = blockIdx.x;
  uint32_t ngroups = gridDim.x;
  if constexpr (FUSE) {
    const uint64_t n_oct = gridDim.x / kNumXcd;
    const uint64_t long_oct = long_groups / kNumXcd;
    const uint64_t oct = blockIdx.x / kNumXcd;
    const uint64_t before = oct * long_oct / n_oct;  // long octets before this one
    const bool is_long = (oct + 1) * long_oct / n_oct > before;
    if (is_long) {
      long_pieces<V, I, AUX>(data, indices, x, x_bytes, n_cols, ls_begin, ls_len, ls_slot,
                             ls_slice_begin, ls_partial,
                             static_cast<uint32_t>(before) * kNumXcd + blockIdx.x % kNumXcd,
                             long_groups);
      return;
    }
    gid = static_cast<uint32_t>(oct - before) * kNumXcd + blockIdx.x % kNumXcd;
    ngroups = gridDim.x - long_groups;
  }
  using A = typename V::Acc;
  // A block spans < 2W values; with the 4-aligned start, <= W/2 + 1 quads.
  // The lanes hold the first QPL * 64 of them (W/2 when W >= 128); the one
  // quad that can lie past those is summed by a separate tail step, so the
  // registers of a whole third chunk are not spent on it.
  constexpr int kQuads = W / 2 + 1;
  constexpr int QPL = (W / 2 + kWave - 1) / kWave;
  constexpr int kCap = 4 * kQuads;  // products staged per wave
  __shared__ A lds_prod[kWavesPerGroup][kCap];
  __shared__ int32_t lds_ptr[kWavesPerGroup][kBlockRows + 1];

  const int lane = threadIdx.x % kWave;
  // wave-uniform by construction; readfirstlane lets the compiler keep the
  // block's buffer descriptors in scalar registers
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
  A *prod = lds_prod[wave];
  int32_t *rptr = lds_ptr[wave];
  const uint32_t lim32 = col_limit32(n_cols);

  const uint32_t first = xcd_remap(gid, ngroups);
  for (int64_t wg = first; wg * kWavesPerGroup < n_bounds; wg += ngroups) {
    const int64_t b = wg * kWavesPerGroup + wave;
    if (b >= n_bounds) break;
    const uint32_t e0 = static_cast<uint32_t>(bounds[b]);
    if (e0 & 0x80000000u) continue;  // long row: summed by spmv_long
    const int64_t r0 = e0;
    const int64_t r1 = static_cast<uint32_t>(bounds[b + 1]) & 0x7fffffffu;
    const int m = static_cast<int>(std::min<int64_t>(r1 - r0, kBlockRows));
    const int64_t p0 = clamp64(bounds_nnz[b], 0, nnz);
    const int64_t p1 = clamp64(bounds_nnz[b + 1], p0, std::min<int64_t>(nnz, p0 + 2 * W - 1));
    const int64_t a0 = p0 & ~int64_t{3};
    // The block's values lie at offsets [p0 - a0, p1 - a0) from a0, in nq
    // quads (fewer than W/2 + 2).
    const int nq = static_cast<int>((p1 - a0 + 3) >> 2);

    // Row pointers of the block (lanes past its m + 1 entries read zero
    // through the descriptor); clamped into the block after phase 1.
    const auto rr = make_rsrc(indptr + r0, static_cast<uint64_t>(m + 1) * sizeof(I));
    constexpr int kRpChunks = (kBlockRows + kWave) / kWave;
    I rpv[kRpChunks];
#pragma unroll
    for (int k = 0; k < kRpChunks; ++k)
      rpv[k] = buffer_index<I>(rr, static_cast<uint32_t>(lane + k * kWave) * sizeof(I));

    // Phase 1 over the chunks of 64 quads the block occupies.
    const int nch = std::min(QPL, (nq + kWave - 1) / kWave);
    block_products_n<V, I, W, AUX, QPL>(nch, data, indices, x, a0, p1, n_cols, lim32, x_bytes,
                                        lane, prod);
    if (nq > QPL * kWave) {  // wave-uniform: the block's last quad, one value per lane
      const int q = QPL * kWave;
      const int64_t pos = a0 + 4 * q + lane;
      if (lane < 4) {
        A pv = vzero<A>();
        if (pos >= p0 && pos < p1) {
          const int64_t col = static_cast<int64_t>(indices[pos]);
          if (static_cast<uint64_t>(col) < static_cast<uint64_t>(n_cols))
            pv = vmul<V>(data[pos], x[col]);
        }
        prod[4 * q + lane] = pv;
      }
    }
#pragma unroll
    for (int k = 0; k < kRpChunks; ++k) {
      const int i = lane + k * kWave;
      if (k == 0 || k * kWave <= m) {  // wave-uniform
        if (i <= m) rptr[i] = block_offset(rpv[k], p0, p1, a0);
      }
    }
    wave_lds_sync();

    // Phase 2: row sums from LDS.  One lane per row (stored order) unless
    // the block holds few rows averaging more than 32 values; then L lanes
    // per row and an XOR butterfly.
    int lg = 0;
    if (p1 - p0 > 32 * static_cast<int64_t>(m) && m <= 32) {
      lg = 6;
      while ((m << lg) > kWave) --lg;
    }
    const int L = 1 << lg;
    const int g = lane >> lg;
    const int j = lane & (L - 1);
    for (int i0 = 0; i0 < m; i0 += (kWave >> lg)) {
      const int i = i0 + g;
      A acc = vzero<A>();
      if (i < m) {
        const int s = rptr[i];
        const int e = rptr[i + 1];
        for (int q = s + j; q < e; q += L) acc = vadd(acc, prod[q]);
      }
      for (int d = L >> 1; d >= 1; d >>= 1) acc = vadd(acc, shfl_xor(acc, d));
      if (i < m && j == 0) y[r0 + i] = V::narrow(acc);
    }
    wave_lds_sync();  // LDS is rewritten by the next block of this wave
  }
}

// --------------------------------------------------------------------------
template <class A>
__device__ inline A block_sum(A v, A *lds4) {
  // fixed-order tree: XOR butterfly in each wave, then waves 0..3 in order
#pragma unroll
  for (int d = kWave / 2; d >= 1; d >>= 1) v = vadd(v, shfl_xor(v, d));
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  if (lane == 0) lds4[wave] = v;
  __syncthreads();
  A total = lds4[0];
  for (int w = 1; w < kWavesPerGroup; ++w) total = vadd(total, lds4[w]);
  __syncthreads();
  return total;
}

template <class V, class I, int AUX>
__global__ void __launch_bounds__(kThreads)
    spmv_long(const typename V::Storage *__restrict__ data, const I *__restrict__ indices,
              const I *__restrict__ indptr, const typename V::Storage *__restrict__ x,
              typename V::Storage *__restrict__ y, const int32_t *__restrict__ long_rows,
              const int32_t *__restrict__ long_chunk_begin, const int32_t *__restrict__ chunk_row,
              typename V::Acc *__restrict__ partials, int64_t n_chunks, int64_t nnz,
              int64_t n_cols, int64_t C, uint32_t x_bytes) {
  using S = typename V::Storage;
  using A = typename V::Acc;
  __shared__ A lds4[kWavesPerGroup];
  for (int64_t c = blockIdx.x; c < n_chunks; c += gridDim.x) {
    const int32_t li = chunk_row[c];
    const int64_t row = long_rows[li];
    const int64_t c_first = long_chunk_begin[li];
    const int64_t n_ch = long_chunk_begin[li + 1] - c_first;
    const int64_t rb = clamp64(static_cast<int64_t>(indptr[row]), 0, nnz);
    const int64_t re = clamp64(static_cast<int64_t>(indptr[row + 1]), rb, nnz);
    const int64_t q0 = std::min(rb + (c - c_first) * C, re);
    const int64_t q1 = std::min(q0 + C, re);
    const int64_t a0 = q0 & ~int64_t{3};
    const int nq = static_cast<int>((q1 - a0 + 3) >> 2);
    // The descriptors end at q1: quads past the chunk read zero.
    const auto ri = make_rsrc(indices + a0, static_cast<uint64_t>(q1 - a0) * sizeof(I));
    const auto rd = make_rsrc(data + a0, static_cast<uint64_t>(q1 - a0) * sizeof(S));
    A acc = vzero<A>();
    if (x_bytes != 0) {
      // Two quads per thread and step; their loads and all 8 gathers are
      // unconditional (out-of-range lanes read zero), so a step costs two
      // dependent round trips.  Sums run over q in order, as below.
      const auto rx = make_rsrc(x, x_bytes);
      for (int q = threadIdx.x; q < nq; q += 2 * kThreads) {
        Quad<I> iq[2];
        Quad<S> dq[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const uint32_t qq = static_cast<uint32_t>(q + u * kThreads);
          iq[u] = load_quad<I, AUX>(ri, qq * 4u * sizeof(I));
          dq[u] = load_quad<S, AUX>(rd, qq * 4u * sizeof(S));
        }
        GatherRaw<S> raw[2][4];
        bool ok[2][4];
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int64_t pos = a0 + 4 * (q + u * kThreads) + e;
            const int64_t col = static_cast<int64_t>(iq[u].v[e]);
            ok[u][e] = pos >= q0 && pos < q1 &&
                       static_cast<uint64_t>(col) < static_cast<uint64_t>(n_cols);
            raw[u][e] = gather_raw<S>(rx, x_bytes, static_cast<uint32_t>(col), ok[u][e]);
          }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const A xv = gather_widen<V>(raw[u][e], static_cast<uint32_t>(iq[u].v[e]));
            const A sum = vadd(acc, vmul_acc<V>(xv, dq[u].v[e]));
            acc = ok[u][e] ? sum : acc;
          }
      }
    } else {  // x beyond a descriptor's reach
#pragma unroll 2
      for (int q = threadIdx.x; q < nq; q += kThreads) {
        const Quad<I> iq = load_quad<I, AUX>(ri, static_cast<uint32_t>(q) * 4u * sizeof(I));
        const Quad<S> dq = load_quad<S, AUX>(rd, static_cast<uint32_t>(q) * 4u * sizeof(S));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t pos = a0 + 4 * q + e;
          const int64_t col = static_cast<int64_t>(iq.v[e]);
          if (pos >= q0 && pos < q1 && static_cast<uint64_t>(col) < static_cast<uint64_t>(n_cols))
            acc = vadd(acc, vmul<V>(dq.v[e], x[col]));
        }
      }
    }
    const A total = block_sum(acc, lds4);
    if (threadIdx.x == 0) {
      if (n_ch == 1)
        y[row] = V::narrow(total);
      else
        partials[c] = total;
    }
  }
}

template <class V>
__global__ void __launch_bounds__(kThreads)
    spmv_long_fixup(typename V::Storage *__restrict__ y, const int32_t *__restrict__ long_rows,
                    const int32_t *__restrict__ long_chunk_begin,
                    const typename V::Acc *__restrict__ partials, int64_t n_long) {
  using A = typename V::Acc;
  const int lane = threadIdx.x % kWave;
  const int64_t li = static_cast<int64_t>(blockIdx.x) * kWavesPerGroup + threadIdx.x / kWave;
  if (li >= n_long) return;
  const int64_t c0 = long_chunk_begin[li];
  const int64_t c1 = long_chunk_begin[li + 1];
  if (c1 - c0 <= 1) return;
  A acc = vzero<A>();
  for (int64_t c = c0 + lane; c < c1; c += kWave) acc = vadd(acc, partials[c]);
#pragma unroll
  for (int d = kWave / 2; d >= 1; d >>= 1) acc = vadd(acc, shfl_xor(acc, d));
  if (lane == 0) y[long_rows[li]] = V::narrow(acc);
}

// --------------------------------------------------------------------------
template <class V, class I>
__global__ void __launch_bounds__(kThreads)
    spmv_rowgroup(const typename V::Storage *__restrict__ data, const I *__restrict__ indices,
                  const I *__restrict__ indptr, const typename V::Storage *__restrict__ x,
                  typename V::Storage *__restrict__ y, int64_t n_rows, int64_t nnz,
                  int64_t n_cols, int G) {
  using A = typename V::Acc;
  const int rows_per_group = kThreads / G;
  const int g = threadIdx.x / G;
  const int j = threadIdx.x % G;
  const int64_t n_tiles = (n_rows + rows_per_group - 1) / rows_per_group;
  for (int64_t t = xcd_remap(blockIdx.x, gridDim.x); t < n_tiles; t += gridDim.x) {
    const int64_t row = t * rows_per_group + g;
    A acc = vzero<A>();
    if (row < n_rows) {
      const int64_t s = clamp64(static_cast<int64_t>(indptr[row]), 0, nnz);
      const int64_t e = clamp64(static_cast<int64_t>(indptr[row + 1]), s, nnz);
      // Four values per lane and step in the row's stored order; every load
      // is unconditional (positions past the row read the step's first
      // value, invalid columns read x[0]) and masked afterwards, so a step
      // costs two dependent round trips instead of two per value.
      if (n_cols > 0) {
        for (int64_t q0 = s + j; q0 < e; q0 += 4 * G) {
          I c[4];
          typename V::Storage d[4], xv[4];
          bool ok[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int64_t q = q0 + u * G;
            const int64_t qc = q < e ? q : q0;
            c[u] = indices[qc];
            d[u] = data[qc];
          }
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int64_t col = static_cast<int64_t>(c[u]);
            ok[u] = q0 + u * G < e && static_cast<uint64_t>(col) < static_cast<uint64_t>(n_cols);
            xv[u] = x[ok[u] ? col : 0];
          }
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const A sum = vadd(acc, vmul<V>(d[u], xv[u]));
            acc = ok[u] ? sum : acc;
          }
        }
      }
    }
    for (int d = G >> 1; d >= 1; d >>= 1) acc = vadd(acc, shfl_xor(acc, d));
    if (row < n_rows && j == 0) y[row] = V::narrow(acc);
  }
}

// --------------------------------------------------------------------------
uint32_t grid_for(int64_t tiles) {
  return static_cast<uint32_t>(std::max<int64_t>(1, std::min<int64_t>(tiles, kMaxGrid)));
}

bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

uint32_t gather_bytes(const void *x, int64_t n_cols, size_t elem) {
  const uint64_t b = (static_cast<uint64_t>(n_cols) * elem + 3) & ~uint64_t{3};
  return n_cols > 0 && b <= kGatherMaxBytes && aligned(x, 4) ? static_cast<uint32_t>(b) : 0u;
}

template <class V, class I>
msx_status spmv_typed(int64_t n_rows, int64_t n_cols, int64_t nnz, const void *data_v,
                      const void *indices_v, const void *indptr_v, const void *x_v, void *y_v,
                      const msx_csr_plan *plan, hipStream_t stream) {
  using S = typename V::Storage;
  using A = typename V::Acc;
  const auto *data = static_cast<const S *>(data_v);
  const auto *indices = static_cast<const I *>(indices_v);
  const auto *indptr = static_cast<const I *>(indptr_v);
  const auto *x = static_cast<const S *>(x_v);
  auto *y = static_cast<S *>(y_v);
  // Quad loads of 4 values: require the streams aligned to their quad size
  // (capped at 16 bytes).
  const bool quads_ok = aligned(data, std::min<size_t>(16, 4 * sizeof(S))) &&
                        aligned(indices, std::min<size_t>(16, 4 * sizeof(I)));
  // Misaligned streams cannot use the quad loads of the plan kernels (the
  // long-row kernel reads the caller's arrays even on a sliced plan).
  const bool use_plan = plan != nullptr && quads_ok;
  // Matrices whose value and index streams cannot stay in the Infinity
  // Cache are read with the non-temporal policy (banded 44.7M values, f32:
  // 140 -> 122 us, bf16: 160 -> 147 us); smaller ones stay cache-resident
  // between calls, which the policy would give up (3D Poisson 128^3:
  // 42 -> 47 us).
  const bool stream_nt =
      static_cast<uint64_t>(nnz) * (sizeof(S) + sizeof(I)) > kStreamNtBytes;
  // x through a buffer descriptor when it fits one and is dword-aligned
  // (0: clamped global loads).
  const uint32_t x_bytes = gather_bytes(x, n_cols, sizeof(S));
  if (use_plan && plan->n_panels > 0) {
    MSX_HIP_TRY_ST(launch_spmv_panels(plan, indptr, x, y, stream));
    if (plan->pn_vstart != nullptr) return MSX_OK;  // long rows are in the panel layout too
  } else if (use_plan && plan->n_slices > 0) {
    MSX_HIP_TRY_ST(launch_spmv_sliced(plan, x, y, stream));
  } else if (use_plan) {
    // Sliced long-row pieces ride in the same launch as the short blocks.
    const bool fuse = plan->n_chunks > 0 && plan->ls_units > 0 && x_bytes != 0;
    if (plan->n_bounds > plan->n_long) {
      const int64_t groups = (plan->n_bounds + kWavesPerGroup - 1) / kWavesPerGroup;
      const uint32_t long_groups =
          fuse ? static_cast<uint32_t>(kSlices * std::max<int64_t>(1, std::min<int64_t>(
                     (plan->ls_slice_max + kWavesPerGroup - 1) / kWavesPerGroup, kMaxGrid / 64)))
               : 0u;
      // fused: the short-block workgroups are a multiple of 8 too, so the
      // grid is whole octets
      uint32_t short_groups = std::min(grid_for(groups), kMaxGrid - long_groups);
      if (fuse) short_groups = (short_groups + kNumXcd - 1) / kNumXcd * kNumXcd;
      const dim3 grid(long_groups + short_groups), block(kThreads);
      A *ls_partial = static_cast<A *>(plan->ls_partial);
#define MSX_SPMV_BLOCKS(WV)                                                                   \
  do {                                                                                         \
    if (fuse && stream_nt)                                                                     \
      hipLaunchKernelGGL((spmv_blocks<V, I, WV, kCacheStream, true>), grid, block, 0, stream,   \
                         data, indices, indptr, x, y, plan->bounds, plan->bounds_nnz,          \
                         plan->n_bounds, nnz, n_cols, x_bytes, long_groups, plan->ls_begin,    \
                         plan->ls_len, plan->ls_slot, plan->ls_slice_begin, ls_partial);       \
    else if (fuse)                                                                             \
      hipLaunchKernelGGL((spmv_blocks<V, I, WV, kCacheDefault, true>), grid, block, 0, stream,  \
                         data, indices, indptr, x, y, plan->bounds, plan->bounds_nnz,          \
                         plan->n_bounds, nnz, n_cols, x_bytes, long_groups, plan->ls_begin,    \
                         plan->ls_len, plan->ls_slot, plan->ls_slice_begin, ls_partial);       \
    else if (stream_nt)                                                                        \
      hipLaunchKernelGGL((spmv_blocks<V, I, WV, kCacheStream, false>), grid, block, 0, stream, \
                         data, indices, indptr, x, y, plan->bounds, plan->bounds_nnz,          \
                         plan->n_bounds, nnz, n_cols, x_bytes, 0u, nullptr, nullptr, nullptr,  \
                         nullptr, nullptr);                                                    \
    else                                                                                       \
      hipLaunchKernelGGL((spmv_blocks<V, I, WV, kCacheDefault, false>), grid, block, 0, stream, \
                         data, indices, indptr, x, y, plan->bounds, plan->bounds_nnz,          \
                         plan->n_bounds, nnz, n_cols, x_bytes, 0u, nullptr, nullptr, nullptr,  \
                         nullptr, nullptr);                                                    \
  } while (0)
      switch (plan->block_nnz) {
      case 64: MSX_SPMV_BLOCKS(64); break;
      case 128: MSX_SPMV_BLOCKS(128); break;
      case 256: MSX_SPMV_BLOCKS(256); break;
      case 512: MSX_SPMV_BLOCKS(512); break;
      default: MSX_SPMV_BLOCKS(1024); break;
      }
#undef MSX_SPMV_BLOCKS
      MSX_HIP_TRY(hipGetLastError());
      if (fuse) {
        MSX_HIP_TRY_ST(launch_long_sliced_fixup(plan, y, stream));
        return MSX_OK;
      }
    }
  }
  if (use_plan && plan->n_chunks > 0 && plan->ls_units > 0 && x_bytes != 0) {
    // long rows cut at the XCD column slices (sorted columns, x >= 4 MB)
    MSX_HIP_TRY_ST(launch_long_sliced(plan, data, indices, x, y, x_bytes, stream_nt, stream));
    return MSX_OK;
  }
  if (use_plan) {
    if (plan->n_chunks > 0) {
      auto long_kernel = stream_nt ? spmv_long<V, I, kCacheStream> : spmv_long<V, I, kCacheDefault>;
      hipLaunchKernelGGL(long_kernel, dim3(grid_for(plan->n_chunks)), dim3(kThreads), 0,
                         stream, data, indices, indptr, x, y, plan->long_rows,
                         plan->long_chunk_begin, plan->chunk_row,
                         static_cast<A *>(plan->partials), plan->n_chunks, nnz, n_cols,
                         plan->chunk_nnz, x_bytes);
      MSX_HIP_TRY(hipGetLastError());
      if (plan->n_chunks > plan->n_long) {
        const int64_t groups = (plan->n_long + kWavesPerGroup - 1) / kWavesPerGroup;
        hipLaunchKernelGGL((spmv_long_fixup<V>), dim3(static_cast<uint32_t>(groups)),
                           dim3(kThreads), 0, stream, y, plan->long_rows, plan->long_chunk_begin,
                           static_cast<const A *>(plan->partials), plan->n_long);
        MSX_HIP_TRY(hipGetLastError());
      }
    }
    return MSX_OK;
  }
  // Plan-free: G lanes per row, the power of two at or below the mean row
  // length (1..64).
  const int64_t avg = n_rows > 0 ? nnz / n_rows : 0;
  int G = 1;
  while (G < kWave && 2 * G <= avg) G <<= 1;
  const int64_t tiles = (n_rows + (kThreads / G) - 1) / (kThreads / G);
  hipLaunchKernelGGL((spmv_rowgroup<V, I>), dim3(grid_for(tiles)), dim3(kThreads), 0, stream, data,
                     indices, indptr, x, y, n_rows, nnz, n_cols, G);
  MSX_HIP_TRY(hipGetLastError());
  return MSX_OK;
}

template <class V>
msx_status spmv_vt(msx_itype it, int64_t n_rows, int64_t n_cols, int64_t nnz, const void *data,
                   const void *indices, const void *indptr, const void *x, void *y,
                   const msx_csr_plan *plan, hipStream_t stream) {
  if (it == MSX_I32)
    return spmv_typed<V, int32_t>(n_rows, n_cols, nnz, data, indices, indptr, x, y, plan, stream);
  return spmv_typed<V, int64_t>(n_rows, n_cols, nnz, data, indices, indptr, x, y, plan, stream);
}

}  // namespace

msx_status launch_spmv(msx_vtype vt, msx_itype it, int64_t n_rows, int64_t n_cols, int64_t nnz,
                       const void *data, const void *indices, const void *indptr, const void *x,
                       void *y, const msx_csr_plan *plan, hipStream_t stream) {
  switch (vt) {
  case MSX_F32:
    return spmv_vt<F32>(it, n_rows, n_cols, nnz, data, indices, indptr, x, y, plan, stream);
  case MSX_F16:
    return spmv_vt<F16>(it, n_rows, n_cols, nnz, data, indices, indptr, x, y, plan, stream);
  case MSX_BF16:
    return spmv_vt<BF16>(it, n_rows, n_cols, nnz, data, indices, indptr, x, y, plan, stream);
  case MSX_C64:
    return spmv_vt<C64>(it, n_rows, n_cols, nnz, data, indices, indptr, x, y, plan, stream);
  }
  return fail(MSX_ETYPE, "csr_matvec unsupported value dtype.");
}

}  // namespace msx
