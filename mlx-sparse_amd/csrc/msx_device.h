// msx_device.h - device-side value traits and memory helpers for gfx950.
//
// Value arithmetic follows the reference accumulator rules
// (reference: src/common/common.h:52-79, src/common/metal_common.h:24-52):
//   float32  : multiply and sum in float32;
//   float16  : widen both operands to float32, multiply and sum in float32,
//              round once to float16 (nearest even);
//   bfloat16 : same with bfloat16 storage;
//   complex64: textbook complex product, sum in complex64.
// The library is compiled with -ffp-contract=off, so products and sums are
// rounded separately, as in the reference's CPU kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>
#include <stdint.h>

#include "msx_sparse.h"

namespace msx {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Value traits.  `Storage` is the element type in memory, `Acc` the type sums
// are carried in.

struct F32 {
  using Storage = float;
  using Acc = float;
  static constexpr msx_vtype kType = MSX_F32;
  __device__ static inline Acc widen(Storage v) { return v; }
  __device__ static inline Storage narrow(Acc v) { return v; }
};

__device__ inline float half_bits_to_float(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// Round-to-nearest-even float32 -> binary16 via the hardware conversion
// (v_cvt_f16_f32 rounds to nearest even under the default mode).
__device__ inline uint16_t float_to_half_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

__device__ inline float bf16_bits_to_float(uint16_t b) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even float32 -> bfloat16 on the bit pattern; NaNs stay
// NaN (quiet bit forced).
__device__ inline uint16_t float_to_bf16_bits(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

struct F16 {
  using Storage = uint16_t;
  using Acc = float;
  static constexpr msx_vtype kType = MSX_F16;
  __device__ static inline Acc widen(Storage v) { return half_bits_to_float(v); }
  __device__ static inline Storage narrow(Acc v) { return float_to_half_bits(v); }
};

struct BF16 {
  using Storage = uint16_t;
  using Acc = float;
  static constexpr msx_vtype kType = MSX_BF16;
  __device__ static inline Acc widen(Storage v) { return bf16_bits_to_float(v); }
  __device__ static inline Storage narrow(Acc v) { return float_to_bf16_bits(v); }
};

struct c64 {
  float re, im;
};

struct C64 {
  using Storage = c64;
  using Acc = c64;
  static constexpr msx_vtype kType = MSX_C64;
  __device__ static inline Acc widen(Storage v) { return v; }
  __device__ static inline Storage narrow(Acc v) { return v; }
};

// Product of two stored values in the accumulator type.
template <class V>
__device__ inline typename V::Acc vmul(typename V::Storage a, typename V::Storage b) {
  return V::widen(a) * V::widen(b);
}
template <>
__device__ inline c64 vmul<C64>(c64 a, c64 b) {
  const float rr = a.re * b.re;
  const float ii = a.im * b.im;
  const float ri = a.re * b.im;
  const float ir = a.im * b.re;
  return c64{rr - ii, ri + ir};
}

// Product of a widened matrix value and a stored RHS value.
template <class V>
__device__ inline typename V::Acc vmul_acc(typename V::Acc a, typename V::Storage b) {
  return a * V::widen(b);
}
template <>
__device__ inline c64 vmul_acc<C64>(c64 a, c64 b) {
  return vmul<C64>(a, b);
}

__device__ inline float vadd(float a, float b) { return a + b; }

// acc + a * x with the reference's rounding (the product rounded to the
// accumulator type, then added).  float16: the product of two binary16
// values has at most 22 significant bits and an exponent inside binary32's
// normal range, so it is exact in float32 and one fused multiply-add gives
// the same bits; gfx950 does it in one v_fma_mix_f32 that also widens x.
template <class V>
__device__ inline typename V::Acc vmadd(typename V::Acc acc, typename V::Acc a,
                                        typename V::Storage x);
__device__ inline c64 vadd(c64 a, c64 b) { return c64{a.re + b.re, a.im + b.im}; }

template <class V>
__device__ inline typename V::Acc vmadd(typename V::Acc acc, typename V::Acc a,
                                        typename V::Storage x) {
  return vadd(acc, vmul_acc<V>(a, x));
}
template <>
__device__ inline float vmadd<F16>(float acc, float a, uint16_t x) {
  return __builtin_fmaf(a, half_bits_to_float(x), acc);
}

template <class A>
__device__ inline A vzero() {
  return A{};
}

// XOR butterfly exchange inside a wavefront.
__device__ inline float shfl_xor(float v, int m) { return __shfl_xor(v, m, kWave); }
__device__ inline c64 shfl_xor(c64 v, int m) {
  return c64{__shfl_xor(v.re, m, kWave), __shfl_xor(v.im, m, kWave)};
}

// ---------------------------------------------------------------------------
// Buffer resources.  A raw buffer descriptor bounds every load to
// [base, base + num_bytes): out-of-range lanes read zero instead of faulting,
// which lets the edge chunks of a row block use full-width loads.  The range
// check works on whole dwords - a dword that straddles the end reads as zero
// - so the size is rounded up to a dword.  Callers pass a base aligned to at
// least 4 bytes, so the rounded tail lies in the same aligned dword as the
// last valid byte (never another page); the kernels mask elements past the
// end themselves.

constexpr int kBufferFlags = 0x00020000;  // gfx9 raw-buffer dword3

__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint64_t num_bytes) {
  num_bytes = (num_bytes + 3) & ~uint64_t{3};
  const uint32_t n = num_bytes > 0xfffffffcull ? 0xfffffffcu : static_cast<uint32_t>(num_bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0),
                                           static_cast<int>(n), kBufferFlags);
}

// Gathers through a descriptor over x.  `x_bytes` is x's size rounded up to
// a dword (at most kGatherMaxBytes); a lane whose element is invalid loads
// from offset x_bytes, past the buffer, and reads zero.  The load therefore
// needs no branch: a conditional load per gather makes the compiler wait for
// each one before issuing the next.  16-bit elements are read as the aligned
// dword that holds them (x is then 4-byte aligned), so each gather fills its
// own 32-bit register.
constexpr uint64_t kGatherMaxBytes = 0xfffffff0ull;

// 0 <= col < n_cols.  An int32 column compares as unsigned against
// lim32 = col_limit32(n_cols) = min(n_cols, 2^31), which also rejects
// negative columns; an int64 column compares against n_cols.
__device__ inline bool col_ok(int32_t col, int64_t, uint32_t lim32) {
  return static_cast<uint32_t>(col) < lim32;
}
__device__ inline bool col_ok(int64_t col, int64_t n_cols, uint32_t) {
  return static_cast<uint64_t>(col) < static_cast<uint64_t>(n_cols);
}
__host__ __device__ inline uint32_t col_limit32(int64_t n_cols) {
  return n_cols >= 0x80000000LL ? 0x80000000u : (n_cols > 0 ? static_cast<uint32_t>(n_cols) : 0u);
}

// Raw bits of x[col] (the holding dword for 16-bit elements), zero when !ok.
template <class S>
using GatherRaw = typename std::conditional<sizeof(S) == 8, uint64_t, uint32_t>::type;

template <class S>
__device__ inline GatherRaw<S> gather_raw(__amdgpu_buffer_rsrc_t rx, uint32_t x_bytes,
                                          uint32_t col, bool ok) {
  if constexpr (sizeof(S) == 2) {
    return __builtin_amdgcn_raw_buffer_load_b32(rx, ok ? (col * 2u) & ~3u : x_bytes, 0, 0);
  } else if constexpr (sizeof(S) == 4) {
    return __builtin_amdgcn_raw_buffer_load_b32(rx, ok ? col * 4u : x_bytes, 0, 0);
  } else {
    const auto w = __builtin_amdgcn_raw_buffer_load_b64(rx, ok ? col * 8u : x_bytes, 0, 0);
    return static_cast<uint64_t>(w[0]) | (static_cast<uint64_t>(w[1]) << 32);
  }
}

// The accumulator value of a gathered element.
template <class V>
__device__ inline typename V::Acc gather_widen(GatherRaw<typename V::Storage> raw, uint32_t col) {
  using S = typename V::Storage;
  if constexpr (sizeof(S) == 2) {
    return V::widen(static_cast<S>(raw >> ((col & 1u) * 16u)));
  } else {
    return V::widen(__builtin_bit_cast(S, raw));
  }
}

// One index (int32 or int64) at byte offset `off` of a buffer; zero past it.
template <class I>
__device__ inline I buffer_index(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  if constexpr (sizeof(I) == 4) {
    return static_cast<I>(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
  } else {
    const auto w = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    return static_cast<I>(static_cast<uint64_t>(w[0]) | (static_cast<uint64_t>(w[1]) << 32));
  }
}

// Cache policy of a buffer load: kCacheDefault, or kCacheStream for data
// read once per call (the non-temporal bit, so it does not displace reused
// lines from L2).
constexpr int kCacheDefault = 0;
constexpr int kCacheStream = 2;
// Matrix streams above this size are read with kCacheStream: they cannot
// stay in MI355X's 256 MB Infinity Cache (memory-side, shared by all XCDs)
// next to x, y and the plan between calls.  Three quarters of the cache.
constexpr uint64_t kStreamNtBytes = uint64_t{192} << 20;

// Load N bytes (8, 16 or 32) at byte offset `off` from a buffer.
template <int N, int AUX = kCacheDefault>
struct BufLoad;

template <int AUX>
struct BufLoad<8, AUX> {
  using T = uint64_t;
  __device__ static inline T load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, AUX);
    return static_cast<uint64_t>(v[0]) | (static_cast<uint64_t>(v[1]) << 32);
  }
};

struct u32x4 {
  uint32_t w[4];
};
struct u32x8 {
  uint32_t w[8];
};

template <int AUX>
struct BufLoad<16, AUX> {
  using T = u32x4;
  __device__ static inline T load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX);
    return u32x4{{v[0], v[1], v[2], v[3]}};
  }
};

template <int AUX>
struct BufLoad<32, AUX> {
  using T = u32x8;
  __device__ static inline T load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    auto a = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX);
    auto b = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16, 0, AUX);
    return u32x8{{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]}};
  }
};

// Four consecutive elements of type E loaded as one vector from a buffer and
// unpacked.
template <class E>
struct Quad {
  E v[4];
};

template <class E, int AUX = kCacheDefault>
__device__ inline Quad<E> load_quad(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  static_assert(sizeof(E) == 2 || sizeof(E) == 4 || sizeof(E) == 8, "element size");
  auto raw = BufLoad<4 * sizeof(E), AUX>::load(r, byte_off);
  return __builtin_bit_cast(Quad<E>, raw);
}

// ---------------------------------------------------------------------------
// XCD-aware workgroup order.  The hardware hands workgroups to the 8 XCDs
// round-robin (workgroup b runs on XCD b % 8).  Remapping b so each XCD
// receives one contiguous run of logical tiles keeps neighbouring rows, and
// the x / X entries they share, in one XCD's L2.
constexpr int kNumXcd = 8;

__device__ inline uint32_t xcd_remap(uint32_t b, uint32_t grid) {
  const uint32_t q = grid / kNumXcd;
  const uint32_t r = grid % kNumXcd;
  const uint32_t xcd = b % kNumXcd;
  const uint32_t slot = b / kNumXcd;
  return xcd * q + (xcd < r ? xcd : r) + slot;
}

}  // namespace msx
