// msx_long_slice.h - the XCD-sliced long-row piece sum, shared by its own
// kernel (csr_long_slice.hip) and the fused short-block kernel
// (csr_spmv.hip).  Long row pieces: see csr_long_slice.hip.
#pragma once

#include <hip/hip_runtime.h>

#include "msx_device.h"
#include "msx_internal.h"

namespace msx {

// A piece starts anywhere, so with its 4-aligned start it spans at most
// kLongPieceMax + 3 positions: 256 quads, four per lane.
constexpr int kLongPieceMax = 1020;
constexpr int kPieceQuads = 4;
constexpr int kLongWavesPerGroup = 4;  // 256-thread workgroups

// Workgroup `gid` of `ngroups` (a multiple of kSlices; workgroup g runs on
// XCD g % 8): its waves sum the pieces of slice gid % 8, one wave per piece
// (quads of 4 values per lane, every load unconditional, then a
// fixed-order butterfly), each into the piece's slot.
template <class V, class I, int AUX>
__device__ __attribute__((always_inline)) inline void long_pieces(const typename V::Storage *__restrict__ data,
                                   const I *__restrict__ indices,
                                   const typename V::Storage *__restrict__ x, uint32_t x_bytes,
                                   int64_t n_cols, const int64_t *__restrict__ ls_begin,
                                   const int32_t *__restrict__ ls_len,
                                   const int32_t *__restrict__ ls_slot,
                                   const int32_t *__restrict__ ls_slice_begin,
                                   typename V::Acc *__restrict__ partial, uint32_t gid,
                                   uint32_t ngroups) {
  using S = typename V::Storage;
  using A = typename V::Acc;
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
  const int s = static_cast<int>(gid % kSlices);  // this workgroup's XCD
  const int64_t u1 = ls_slice_begin[s + 1];
  const int64_t step = static_cast<int64_t>(ngroups / kSlices) * kLongWavesPerGroup;
  const auto rx = make_rsrc(x, x_bytes);
  const uint32_t lim32 = col_limit32(n_cols);
  for (int64_t u = ls_slice_begin[s] + static_cast<int64_t>(gid / kSlices) * kLongWavesPerGroup + wave;
       u < u1; u += step) {
    const int64_t pb = ls_begin[u];
    const int64_t pe = pb + ls_len[u];
    const int64_t a0 = pb & ~int64_t{3};
    // descriptors end at the piece: later quads read zero
    const auto ri = make_rsrc(indices + a0, static_cast<uint64_t>(pe - a0) * sizeof(I));
    const auto rd = make_rsrc(data + a0, static_cast<uint64_t>(pe - a0) * sizeof(S));
    Quad<I> iq[kPieceQuads];
    Quad<S> dq[kPieceQuads];
#pragma unroll
    for (int j = 0; j < kPieceQuads; ++j) {
      const uint32_t q = static_cast<uint32_t>(lane + j * kWave);
      iq[j] = load_quad<I, AUX>(ri, q * 4u * sizeof(I));
      dq[j] = load_quad<S, AUX>(rd, q * 4u * sizeof(S));
    }
    // positions as offsets from a0: the piece is [lo, hi), hi <= 1023
    const uint32_t lo = static_cast<uint32_t>(pb - a0);
    const uint32_t span = static_cast<uint32_t>(pe - pb);
    GatherRaw<S> raw[kPieceQuads][4];
    bool ok[kPieceQuads][4];
#pragma unroll
    for (int j = 0; j < kPieceQuads; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t off = 4u * static_cast<uint32_t>(lane + j * kWave) + e;
        const I col = iq[j].v[e];
        ok[j][e] = off - lo < span && col_ok(col, n_cols, lim32);
        raw[j][e] = gather_raw<S>(rx, x_bytes, static_cast<uint32_t>(col), ok[j][e]);
      }
    __builtin_amdgcn_sched_barrier(0);
    A acc = vzero<A>();
#pragma unroll
    for (int j = 0; j < kPieceQuads; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const A xv = gather_widen<V>(raw[j][e], static_cast<uint32_t>(iq[j].v[e]));
        const A sum = vadd(acc, vmul_acc<V>(xv, dq[j].v[e]));
        acc = ok[j][e] ? sum : acc;
      }
#pragma unroll
    for (int d = kWave / 2; d >= 1; d >>= 1) acc = vadd(acc, shfl_xor(acc, d));
    if (lane == 0) partial[ls_slot[u]] = acc;
  }
}

}  // namespace msx
