// csr_cpu.cpp - host SpMV / SpMM for the `use_cpu()` device.
//
// Restates the reference CPU backend on plain host pointers:
//   - rows summed sequentially in stored order in the accumulator type;
//     SpMV rows of length 1..4 start from their first product, longer rows
//     from zero (reference: src/sparse/csr_matvec/csr_matvec.cpp:79-114);
//   - SpMM keeps one accumulator per RHS column and sums each from zero in
//     stored order (reference: src/sparse/csr_matmul/csr_matmul.cpp:83-133);
//   - per call: an O(n) row-work prepass, contiguous work-balanced row ranges
//     and one std::thread per extra range, the first exception rethrown on
//     the caller (reference: csr_matvec.cpp:116-168, csr_matmul.cpp:172-222,
//     src/common/cpu_parallel.h:50-164, src/common/cpu_parallel.cpp:97-253).
// Threads own disjoint rows, so the output does not depend on the thread
// count.  Compiled without -ffp-contract: every product and sum is rounded
// on its own.
#include <sched.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <exception>
#include <limits>
#include <mutex>
#include <new>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "msx_sparse.h"

namespace msx {
msx_status fail(msx_status code, const std::string &msg);
void clear_error();
}  // namespace msx

namespace msx {
namespace cpu {
namespace {

// ---------------------------------------------------------------------------
// Value types on the host.

struct cf32 {
  float re, im;
};

inline float bits_to_float(uint32_t u) {
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
}
inline uint32_t float_to_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, sizeof u);
  return u;
}

// binary16 -> binary32, exact.
float half_to_float(uint16_t h) {
  const uint32_t s = static_cast<uint32_t>(h >> 15) << 31;
  const uint32_t e = (h >> 10) & 31u;
  const uint32_t m = h & 1023u;
  if (e == 31) return bits_to_float(s | 0x7f800000u | (m << 13));
  if (e != 0) return bits_to_float(s | ((e + 112u) << 23) | (m << 13));
  if (m == 0) return bits_to_float(s);
  // subnormal: normalise the significand
  int shift = 0;
  uint32_t mm = m;
  while ((mm & 1024u) == 0) {
    mm <<= 1;
    ++shift;
  }
  return bits_to_float(s | ((113u - shift) << 23) | ((mm & 1023u) << 13));
}

// binary32 -> binary16, round to nearest even.  Works on the magnitude in
// units of the target's last place: the binary16 grid below 2^-14 is uniform
// (2^-24 steps), above it the exponent field is rebased.
uint16_t float_to_half(float f) {
  const uint32_t u = float_to_bits(f);
  const uint16_t s = static_cast<uint16_t>((u >> 16) & 0x8000u);
  const uint32_t a = u & 0x7fffffffu;
  if (a >= 0x7f800000u) return static_cast<uint16_t>(s | (a > 0x7f800000u ? 0x7e00u : 0x7c00u));
  const int e = static_cast<int>(a >> 23) - 127;
  if (e >= 16) return static_cast<uint16_t>(s | 0x7c00u);
  uint32_t sig = (a & 0x7fffffu) | (a >= 0x00800000u ? 0x800000u : 0u);
  // number of low bits of the 24-bit significand that fall below the
  // binary16 last place at this exponent
  int drop = e < -14 ? (13 + (-14 - e)) : 13;
  if (a < 0x00800000u) drop = 13 + 14 + 112;  // binary32 subnormal: far below 2^-24
  if (drop > 31) return s;
  uint32_t q = sig >> drop;
  const uint32_t rem = sig & ((1u << drop) - 1u);
  const uint32_t half = 1u << (drop - 1);
  if (rem > half || (rem == half && (q & 1u))) ++q;
  if (e < -14) return static_cast<uint16_t>(s | q);  // subnormal (q may round up to 0x400)
  // normal: q holds the implicit bit at 2^10; carry may bump the exponent
  const uint32_t biased = static_cast<uint32_t>(e + 15);
  const uint32_t out = (biased << 10) + (q - 1024u);
  return static_cast<uint16_t>(s | std::min<uint32_t>(out, 0x7c00u));
}

float bf16_to_float(uint16_t b) { return bits_to_float(static_cast<uint32_t>(b) << 16); }

uint16_t float_to_bf16(float f) {
  uint32_t u = float_to_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

struct F32 {
  using S = float;
  using A = float;
  static A widen(S v) { return v; }
  static S narrow(A v) { return v; }
  static A mul(S a, S b) { return a * b; }
};
struct F16 {
  using S = uint16_t;
  using A = float;
  static A widen(S v) { return half_to_float(v); }
  static S narrow(A v) { return float_to_half(v); }
  static A mul(S a, S b) { return half_to_float(a) * half_to_float(b); }
};
struct BF16 {
  using S = uint16_t;
  using A = float;
  static A widen(S v) { return bf16_to_float(v); }
  static S narrow(A v) { return float_to_bf16(v); }
  static A mul(S a, S b) { return bf16_to_float(a) * bf16_to_float(b); }
};
struct C64 {
  using S = cf32;
  using A = cf32;
  static A widen(S v) { return v; }
  static S narrow(A v) { return v; }
  static A mul(S a, S b) {
    const float rr = a.re * b.re, ii = a.im * b.im, ri = a.re * b.im, ir = a.im * b.re;
    return cf32{rr - ii, ri + ir};
  }
};

inline float add(float a, float b) { return a + b; }
inline cf32 add(cf32 a, cf32 b) { return cf32{a.re + b.re, a.im + b.im}; }

// ---------------------------------------------------------------------------
// Worker count and ranges.

int parse_positive(const char *v) {
  if (v == nullptr || *v == '\0') return 0;
  char *end = nullptr;
  const long x = std::strtol(v, &end, 10);
  if (end == v || x <= 0 || x > std::numeric_limits<int>::max()) return 0;
  if (*end != '\0' && *end != ',') return 0;
  return static_cast<int>(x);
}

int auto_workers() {
  if (int c = parse_positive(std::getenv("OMP_NUM_THREADS")); c > 0) return c;
  for (const char *name : {"SLURM_CPUS_PER_TASK", "PBS_NP", "LSB_DJOB_NUMPROC", "NSLOTS"})
    if (int c = parse_positive(std::getenv(name)); c > 0) return c;
  cpu_set_t set;
  CPU_ZERO(&set);
  if (sched_getaffinity(0, sizeof(set), &set) == 0)
    if (int c = CPU_COUNT(&set); c > 0) return c;
  const int hw = static_cast<int>(std::thread::hardware_concurrency());
  return hw > 0 ? hw : 1;
}

struct Range {
  int64_t begin, end;
};

std::vector<Range> equal_ranges(int64_t n, int parts) {
  std::vector<Range> out;
  if (n <= 0) return out;
  const int count = std::max(1, parts);
  for (int p = 0; p < count; ++p) {
    const int64_t b = (static_cast<int64_t>(p) * n) / count;
    const int64_t e = (static_cast<int64_t>(p + 1) * n) / count;
    if (b < e) out.push_back({b, e});
  }
  return out;
}

std::vector<Range> weighted_ranges(const std::vector<int64_t> &work, int parts) {
  const int64_t n = static_cast<int64_t>(work.size());
  if (n <= 0) return {};
  const int count = std::max(1, parts);
  if (count == 1) return {{0, n}};
  if (count >= n) return equal_ranges(n, count);
  std::vector<int64_t> prefix(static_cast<size_t>(n) + 1, 0);
  for (int64_t r = 0; r < n; ++r) {
    const int64_t next = prefix[r] + std::max<int64_t>(0, work[r]);
    prefix[r + 1] = next < prefix[r] ? std::numeric_limits<int64_t>::max() : next;
  }
  if (prefix.back() <= 0) return equal_ranges(n, count);
  std::vector<Range> out;
  int64_t begin = 0;
  for (int part = 0; part < count && begin < n; ++part) {
    const int left = count - part;
    if (left == 1) {
      out.push_back({begin, n});
      break;
    }
    const int64_t target = prefix[begin] + (prefix.back() - prefix[begin] + left - 1) / left;
    int64_t end = std::lower_bound(prefix.begin() + begin + 1, prefix.end(), target) - prefix.begin();
    end = std::max(end, begin + 1);
    end = std::min(end, n - (left - 1));
    out.push_back({begin, end});
    begin = end;
  }
  return out;
}

std::vector<Range> ranges_for_work(const std::vector<int64_t> &work, int parts) {
  if (work.empty()) return {};
  const int64_t n = static_cast<int64_t>(work.size());
  if (parts <= 1) return {{0, n}};
  bool uneven = false;
  for (size_t i = 1; i < work.size() && !uneven; ++i)
    uneven = std::max<int64_t>(0, work[i]) != std::max<int64_t>(0, work[i - 1]);
  return uneven ? weighted_ranges(work, parts) : equal_ranges(n, parts);
}

template <class Fn>
void parallel_for(const std::vector<Range> &ranges, Fn &&fn) {
  if (ranges.empty()) return;
  if (ranges.size() == 1) {
    fn(ranges[0]);
    return;
  }
  std::atomic<bool> failed{false};
  std::exception_ptr first = nullptr;
  auto run = [&](Range r) {
    if (failed.load(std::memory_order_relaxed)) return;
    try {
      fn(r);
    } catch (...) {
      bool expected = false;
      if (failed.compare_exchange_strong(expected, true)) first = std::current_exception();
    }
  };
  std::vector<std::thread> threads;
  threads.reserve(ranges.size() - 1);
  for (size_t i = 1; i < ranges.size(); ++i) threads.emplace_back(run, ranges[i]);
  run(ranges[0]);
  for (auto &t : threads) t.join();
  if (first) std::rethrow_exception(first);
}

// ---------------------------------------------------------------------------
// Kernels.

template <class I>
inline int64_t at(const I *p, int64_t i) {
  return static_cast<int64_t>(p[i]);
}

template <class V, class I>
void spmv_rows(const typename V::S *data, const I *indices, const I *indptr,
               const typename V::S *x, typename V::S *y, Range r) {
  using A = typename V::A;
  for (int64_t row = r.begin; row < r.end; ++row) {
    const int64_t b = at(indptr, row), e = at(indptr, row + 1);
    A acc{};
    int64_t p = b;
    if (e - b >= 1 && e - b <= 4) {
      acc = V::mul(data[p], x[at(indices, p)]);
      ++p;
    }
    for (; p < e; ++p) acc = add(acc, V::mul(data[p], x[at(indices, p)]));
    y[row] = V::narrow(acc);
  }
}

template <class V, class I>
void spmm_rows(const typename V::S *data, const I *indices, const I *indptr,
               const typename V::S *X, typename V::S *Y, int64_t k, Range r) {
  using A = typename V::A;
  std::vector<A> acc(static_cast<size_t>(std::max<int64_t>(k, 1)));
  for (int64_t row = r.begin; row < r.end; ++row) {
    std::fill(acc.begin(), acc.end(), A{});
    for (int64_t p = at(indptr, row); p < at(indptr, row + 1); ++p) {
      const typename V::S v = data[p];
      const typename V::S *xr = X + at(indices, p) * k;
      for (int64_t c = 0; c < k; ++c) acc[c] = add(acc[c], V::mul(v, xr[c]));
    }
    for (int64_t c = 0; c < k; ++c) Y[row * k + c] = V::narrow(acc[c]);
  }
}

template <class I>
std::vector<int64_t> row_work(const I *indptr, int64_t n, int64_t scale) {
  std::vector<int64_t> w(static_cast<size_t>(n));
  for (int64_t r = 0; r < n; ++r) w[r] = (at(indptr, r + 1) - at(indptr, r)) * scale;
  return w;
}

template <class V, class I>
void spmv(int64_t n, const void *data, const void *indices, const void *indptr, const void *x,
          void *y, int workers) {
  const auto *d = static_cast<const typename V::S *>(data);
  const auto *ix = static_cast<const I *>(indices);
  const auto *ip = static_cast<const I *>(indptr);
  const auto *xv = static_cast<const typename V::S *>(x);
  auto *yv = static_cast<typename V::S *>(y);
  auto body = [&](Range r) { spmv_rows<V, I>(d, ix, ip, xv, yv, r); };
  if (workers <= 1 || n <= 0) return body({0, n});
  const auto ranges = ranges_for_work(row_work(ip, n, 1), workers);
  if (ranges.size() <= 1) return body({0, n});
  parallel_for(ranges, body);
}

template <class V, class I>
void spmm(int64_t n, int64_t k, const void *data, const void *indices, const void *indptr,
          const void *X, void *Y, int workers) {
  const auto *d = static_cast<const typename V::S *>(data);
  const auto *ix = static_cast<const I *>(indices);
  const auto *ip = static_cast<const I *>(indptr);
  const auto *xv = static_cast<const typename V::S *>(X);
  auto *yv = static_cast<typename V::S *>(Y);
  auto body = [&](Range r) { spmm_rows<V, I>(d, ix, ip, xv, yv, k, r); };
  if (workers <= 1 || n <= 0) return body({0, n});
  const auto ranges = ranges_for_work(row_work(ip, n, std::max<int64_t>(k, 1)), workers);
  if (ranges.size() <= 1) return body({0, n});
  parallel_for(ranges, body);
}

// Batched: items (b, row), b < batch; batch b reads X + b * n_cols * k and
// writes Y + b * n_rows * k.  Work per item = row length * max(k, 1).
template <class V, class I>
void batched(int64_t n, int64_t n_cols, int64_t batch, int64_t k, const void *data,
             const void *indices, const void *indptr, const void *X, void *Y, int workers) {
  const auto *d = static_cast<const typename V::S *>(data);
  const auto *ix = static_cast<const I *>(indices);
  const auto *ip = static_cast<const I *>(indptr);
  const auto *xv = static_cast<const typename V::S *>(X);
  auto *yv = static_cast<typename V::S *>(Y);
  using A = typename V::A;
  const int64_t items = n * batch;
  auto body = [&](Range r) {
    std::vector<A> acc(static_cast<size_t>(std::max<int64_t>(k, 1)));
    for (int64_t item = r.begin; item < r.end; ++item) {
      const int64_t b = item / n, row = item - b * n;
      const typename V::S *xb = xv + b * n_cols * k;
      std::fill(acc.begin(), acc.end(), A{});
      for (int64_t p = at(ip, row); p < at(ip, row + 1); ++p) {
        const typename V::S v = d[p];
        const typename V::S *xr = xb + at(ix, p) * k;
        for (int64_t c = 0; c < k; ++c) acc[c] = add(acc[c], V::mul(v, xr[c]));
      }
      typename V::S *yr = yv + (b * n + row) * k;
      for (int64_t c = 0; c < k; ++c) yr[c] = V::narrow(acc[c]);
    }
  };
  if (workers <= 1 || items <= 0) return body({0, items});
  std::vector<int64_t> work(static_cast<size_t>(items));
  for (int64_t item = 0; item < items; ++item) {
    const int64_t row = item % n;
    work[item] = (at(ip, row + 1) - at(ip, row)) * std::max<int64_t>(k, 1);
  }
  const auto ranges = ranges_for_work(work, workers);
  if (ranges.size() <= 1) return body({0, items});
  parallel_for(ranges, body);
}

// A^T X (k = 1: A^T x) as the reference computes it: serially, each output
// from zero over the rows in order; with several workers, per-partition
// partial outputs (rows split by row length) added from zero in partition
// order.  Columns outside [0, n_cols) add nothing.
template <class V, class I>
void transpose_product(int64_t n_rows, int64_t n_cols, int64_t k, const void *data,
                       const void *indices, const void *indptr, const void *X, void *Y,
                       int workers) {
  const auto *d = static_cast<const typename V::S *>(data);
  const auto *ix = static_cast<const I *>(indices);
  const auto *ip = static_cast<const I *>(indptr);
  const auto *xv = static_cast<const typename V::S *>(X);
  auto *yv = static_cast<typename V::S *>(Y);
  using A = typename V::A;
  const int64_t out_size = n_cols * k;
  auto rows_into = [&](A *acc, Range r) {
    for (int64_t row = r.begin; row < r.end; ++row) {
      const typename V::S *xr = xv + row * k;
      for (int64_t p = at(ip, row); p < at(ip, row + 1); ++p) {
        const int64_t col = at(ix, p);
        if (col < 0 || col >= n_cols) continue;
        for (int64_t q = 0; q < k; ++q) acc[col * k + q] = add(acc[col * k + q], V::mul(d[p], xr[q]));
      }
    }
  };
  std::vector<Range> ranges;
  if (workers > 1 && n_rows > 0 && out_size > 0) ranges = ranges_for_work(row_work(ip, n_rows, 1), workers);
  if (ranges.size() <= 1) {
    std::vector<A> acc(static_cast<size_t>(out_size), A{});
    rows_into(acc.data(), {0, n_rows});
    for (int64_t i = 0; i < out_size; ++i) yv[i] = V::narrow(acc[i]);
    return;
  }
  const size_t parts = ranges.size();
  std::vector<A> partial(parts * static_cast<size_t>(out_size), A{});
  std::vector<Range> indexed = ranges;
  std::vector<std::thread> pool;
  std::exception_ptr err;
  std::mutex mu;
  for (size_t w = 0; w < parts; ++w) {
    pool.emplace_back([&, w] {
      try {
        rows_into(partial.data() + w * out_size, indexed[w]);
      } catch (...) {
        std::lock_guard<std::mutex> lock(mu);
        if (!err) err = std::current_exception();
      }
    });
  }
  for (auto &t : pool) t.join();
  if (err) std::rethrow_exception(err);
  auto reduce = [&](Range r) {
    for (int64_t i = r.begin; i < r.end; ++i) {
      A total{};
      for (size_t w = 0; w < parts; ++w) total = add(total, partial[w * out_size + i]);
      yv[i] = V::narrow(total);
    }
  };
  const auto out_ranges = equal_ranges(out_size, workers);
  if (out_ranges.size() <= 1) return reduce({0, out_size});
  parallel_for(out_ranges, reduce);
}

// CSR of A^T by a counting sort: column counts, prefix, then the rows in
// order, so every column lists its entries by increasing row.
template <class V, class I>
void transpose_csr(int64_t n_rows, int64_t n_cols, int64_t nnz, const void *data,
                   const void *indices, const void *indptr, void *t_data, void *t_indices,
                   void *t_indptr) {
  const auto *d = static_cast<const typename V::S *>(data);
  const auto *ix = static_cast<const I *>(indices);
  const auto *ip = static_cast<const I *>(indptr);
  auto *td = static_cast<typename V::S *>(t_data);
  auto *ti = static_cast<I *>(t_indices);
  auto *tp = static_cast<I *>(t_indptr);
  std::vector<int64_t> next(static_cast<size_t>(n_cols) + 1, 0);
  for (int64_t row = 0; row < n_rows; ++row)
    for (int64_t p = at(ip, row); p < at(ip, row + 1); ++p) {
      const int64_t c = at(ix, p);
      if (c >= 0 && c < n_cols) ++next[c + 1];
    }
  for (int64_t c = 0; c < n_cols; ++c) next[c + 1] += next[c];
  for (int64_t c = 0; c <= n_cols; ++c) tp[c] = static_cast<I>(next[c]);
  for (int64_t row = 0; row < n_rows; ++row)
    for (int64_t p = at(ip, row); p < at(ip, row + 1); ++p) {
      const int64_t c = at(ix, p);
      if (c < 0 || c >= n_cols) continue;
      const int64_t slot = next[c]++;
      td[slot] = d[p];
      ti[slot] = static_cast<I>(row);
    }
  // dropped values (columns out of range): zero bits and row 0 past
  // t_indptr[n_cols] (nnz is the length of the output buffers), the same
  // tail as the GPU transpose writes
  for (int64_t slot = next[n_cols]; slot < nnz; ++slot) {
    memset(&td[slot], 0, sizeof(td[slot]));
    ti[slot] = I(0);
  }
}

// Value gradients: g[p] = sum_q cot[row, q] * X[col, q] from zero, or with
// `single` (the SpMV rule) the one product cot[row] * x[col] - they differ in
// the sign of a zero product.
template <class V, class I>
void data_vjp(int64_t n_rows, int64_t n_cols, int64_t k, bool single, const void *indices,
              const void *indptr, const void *X, const void *cot, void *out, int workers) {
  const auto *ix = static_cast<const I *>(indices);
  const auto *ip = static_cast<const I *>(indptr);
  const auto *xv = static_cast<const typename V::S *>(X);
  const auto *cv = static_cast<const typename V::S *>(cot);
  auto *ov = static_cast<typename V::S *>(out);
  using A = typename V::A;
  auto body = [&](Range r) {
    for (int64_t row = r.begin; row < r.end; ++row) {
      for (int64_t p = at(ip, row); p < at(ip, row + 1); ++p) {
        const int64_t col = at(ix, p);
        A acc{};
        if (col >= 0 && col < n_cols) {
          if (single) {
            acc = V::mul(cv[row], xv[col]);
          } else {
            for (int64_t q = 0; q < k; ++q) acc = add(acc, V::mul(cv[row * k + q], xv[col * k + q]));
          }
        }
        ov[p] = V::narrow(acc);
      }
    }
  };
  if (workers <= 1 || n_rows <= 0) return body({0, n_rows});
  const auto ranges = ranges_for_work(row_work(ip, n_rows, 1), workers);
  if (ranges.size() <= 1) return body({0, n_rows});
  parallel_for(ranges, body);
}

}  // namespace

int worker_count() {
  const char *raw = std::getenv("MLX_SPARSE_CPU_THREADS");
  if (raw == nullptr || *raw == '\0') raw = std::getenv("MLX_SPARSE_N_THREADS");
  if (int c = parse_positive(raw); c > 0) return c;
  return auto_workers();
}

}  // namespace cpu
}  // namespace msx

using namespace msx;

namespace {

msx_status check_cpu(const char *op, msx_vtype vt, msx_itype it, int64_t n_rows, int64_t n_cols,
                     int64_t nnz, const void *data, const void *indices, const void *indptr) {
  if (it != MSX_I32 && it != MSX_I64)
    return fail(MSX_ETYPE, std::string(op) + " requires int32 or int64 indices.");
  if (vt < MSX_F32 || vt > MSX_C64) return fail(MSX_ETYPE, std::string(op) + " unsupported value dtype.");
  if (n_rows < 0 || n_cols < 0 || nnz < 0)
    return fail(MSX_EINVAL, std::string(op) + " shape dimensions must be non-negative.");
  if (indptr == nullptr) return fail(MSX_EINVAL, std::string(op) + " indptr is NULL.");
  if (nnz > 0 && (data == nullptr || indices == nullptr))
    return fail(MSX_EINVAL, std::string(op) + " data and indices must be non-NULL when nnz > 0.");
  return MSX_OK;
}

template <class Fn>
msx_status guarded(const char *op, Fn &&fn) {
  try {
    fn();
  } catch (const std::bad_alloc &) {
    return fail(MSX_ENOMEM, std::string(op) + ": host allocation failed.");
  } catch (const std::exception &e) {
    return fail(MSX_EINVAL, std::string(op) + ": " + e.what());
  }
  return MSX_OK;
}

}  // namespace

extern "C" msx_status msx_csr_spmv_cpu(msx_vtype vt, msx_itype it, int64_t n_rows, int64_t n_cols,
                                       int64_t nnz, const void *data, const void *indices,
                                       const void *indptr, const void *x, void *y, int n_threads) {
  clear_error();
  msx_status st = check_cpu("csr_matvec", vt, it, n_rows, n_cols, nnz, data, indices, indptr);
  if (st != MSX_OK) return st;
  if (n_rows > 0 && y == nullptr) return fail(MSX_EINVAL, "csr_matvec y is NULL.");
  const int workers = n_threads > 0 ? n_threads : cpu::worker_count();
  return guarded("csr_matvec", [&] {
    const bool i64 = it == MSX_I64;
    switch (vt) {
    case MSX_F32:
      i64 ? cpu::spmv<cpu::F32, int64_t>(n_rows, data, indices, indptr, x, y, workers)
          : cpu::spmv<cpu::F32, int32_t>(n_rows, data, indices, indptr, x, y, workers);
      break;
    case MSX_F16:
      i64 ? cpu::spmv<cpu::F16, int64_t>(n_rows, data, indices, indptr, x, y, workers)
          : cpu::spmv<cpu::F16, int32_t>(n_rows, data, indices, indptr, x, y, workers);
      break;
    case MSX_BF16:
      i64 ? cpu::spmv<cpu::BF16, int64_t>(n_rows, data, indices, indptr, x, y, workers)
          : cpu::spmv<cpu::BF16, int32_t>(n_rows, data, indices, indptr, x, y, workers);
      break;
    case MSX_C64:
      i64 ? cpu::spmv<cpu::C64, int64_t>(n_rows, data, indices, indptr, x, y, workers)
          : cpu::spmv<cpu::C64, int32_t>(n_rows, data, indices, indptr, x, y, workers);
      break;
    }
  });
}

extern "C" msx_status msx_csr_spmm_cpu(msx_vtype vt, msx_itype it, int64_t n_rows, int64_t n_cols,
                                       int64_t nnz, const void *data, const void *indices,
                                       const void *indptr, int64_t k, const void *X, void *Y,
                                       int n_threads) {
  clear_error();
  msx_status st = check_cpu("csr_matmul", vt, it, n_rows, n_cols, nnz, data, indices, indptr);
  if (st != MSX_OK) return st;
  if (k < 0) return fail(MSX_EINVAL, "csr_matmul rhs column count must be non-negative.");
  if (n_rows > 0 && k > 0 && Y == nullptr) return fail(MSX_EINVAL, "csr_matmul Y is NULL.");
  const int workers = n_threads > 0 ? n_threads : cpu::worker_count();
  return guarded("csr_matmul", [&] {
    const bool i64 = it == MSX_I64;
    switch (vt) {
    case MSX_F32:
      i64 ? cpu::spmm<cpu::F32, int64_t>(n_rows, k, data, indices, indptr, X, Y, workers)
          : cpu::spmm<cpu::F32, int32_t>(n_rows, k, data, indices, indptr, X, Y, workers);
      break;
    case MSX_F16:
      i64 ? cpu::spmm<cpu::F16, int64_t>(n_rows, k, data, indices, indptr, X, Y, workers)
          : cpu::spmm<cpu::F16, int32_t>(n_rows, k, data, indices, indptr, X, Y, workers);
      break;
    case MSX_BF16:
      i64 ? cpu::spmm<cpu::BF16, int64_t>(n_rows, k, data, indices, indptr, X, Y, workers)
          : cpu::spmm<cpu::BF16, int32_t>(n_rows, k, data, indices, indptr, X, Y, workers);
      break;
    case MSX_C64:
      i64 ? cpu::spmm<cpu::C64, int64_t>(n_rows, k, data, indices, indptr, X, Y, workers)
          : cpu::spmm<cpu::C64, int32_t>(n_rows, k, data, indices, indptr, X, Y, workers);
      break;
    }
  });
}

extern "C" int msx_cpu_worker_count(void) { return cpu::worker_count(); }

extern "C" msx_status msx_cpu_ranges(const int64_t *work, int64_t n, int parts, int64_t *ranges,
                                     int64_t *n_ranges) {
  clear_error();
  if (n < 0 || (n > 0 && work == nullptr) || ranges == nullptr || n_ranges == nullptr)
    return fail(MSX_EINVAL, "msx_cpu_ranges: invalid arguments.");
  return guarded("msx_cpu_ranges", [&] {
    std::vector<int64_t> w(work, work + n);
    const auto r = cpu::ranges_for_work(w, parts);
    for (size_t i = 0; i < r.size(); ++i) {
      ranges[2 * i] = r[i].begin;
      ranges[2 * i + 1] = r[i].end;
    }
    *n_ranges = static_cast<int64_t>(r.size());
  });
}

namespace {

template <class V>
void batched_vt(msx_itype it, int64_t n_rows, int64_t n_cols, int64_t batch, int64_t k,
                const void *data, const void *indices, const void *indptr, const void *X, void *Y,
                int workers) {
  if (it == MSX_I64)
    cpu::batched<V, int64_t>(n_rows, n_cols, batch, k, data, indices, indptr, X, Y, workers);
  else
    cpu::batched<V, int32_t>(n_rows, n_cols, batch, k, data, indices, indptr, X, Y, workers);
}

msx_status batched_cpu(const char *op, msx_vtype vt, msx_itype it, int64_t n_rows, int64_t n_cols,
                       int64_t nnz, const void *data, const void *indices, const void *indptr,
                       int64_t batch, int64_t k, const void *X, void *Y, int n_threads) {
  clear_error();
  msx_status st = check_cpu(op, vt, it, n_rows, n_cols, nnz, data, indices, indptr);
  if (st != MSX_OK) return st;
  if (batch < 0 || k < 0) return fail(MSX_EINVAL, std::string(op) + " shape dimensions must be non-negative.");
  if (batch > 0 && n_rows > 0 && k > 0 && Y == nullptr)
    return fail(MSX_EINVAL, std::string(op) + " Y is NULL.");
  if (batch > 0 && n_cols > 0 && k > 0 && nnz > 0 && X == nullptr)
    return fail(MSX_EINVAL, std::string(op) + " X is NULL.");
  if (batch == 0 || n_rows == 0 || k == 0) return MSX_OK;
  const int workers = n_threads > 0 ? n_threads : cpu::worker_count();
  return guarded(op, [&] {
    switch (vt) {
    case MSX_F32: batched_vt<cpu::F32>(it, n_rows, n_cols, batch, k, data, indices, indptr, X, Y, workers); break;
    case MSX_F16: batched_vt<cpu::F16>(it, n_rows, n_cols, batch, k, data, indices, indptr, X, Y, workers); break;
    case MSX_BF16: batched_vt<cpu::BF16>(it, n_rows, n_cols, batch, k, data, indices, indptr, X, Y, workers); break;
    case MSX_C64: batched_vt<cpu::C64>(it, n_rows, n_cols, batch, k, data, indices, indptr, X, Y, workers); break;
    }
  });
}

}  // namespace

extern "C" msx_status msx_csr_batched_spmv_cpu(msx_vtype vt, msx_itype it, int64_t n_rows,
                                               int64_t n_cols, int64_t nnz, const void *data,
                                               const void *indices, const void *indptr,
                                               int64_t batch, const void *X, void *Y,
                                               int n_threads) {
  return batched_cpu("csr_batched_matvec", vt, it, n_rows, n_cols, nnz, data, indices, indptr,
                     batch, 1, X, Y, n_threads);
}

extern "C" msx_status msx_csr_batched_spmm_cpu(msx_vtype vt, msx_itype it, int64_t n_rows,
                                               int64_t n_cols, int64_t nnz, const void *data,
                                               const void *indices, const void *indptr,
                                               int64_t batch, int64_t k, const void *X, void *Y,
                                               int n_threads) {
  return batched_cpu("csr_batched_matmul", vt, it, n_rows, n_cols, nnz, data, indices, indptr,
                     batch, k, X, Y, n_threads);
}

namespace {

template <template <class, class> class Fn, class... Args>
void dispatch_cpu(msx_vtype vt, msx_itype it, Args... args) {
  const bool i64 = it == MSX_I64;
  switch (vt) {
  case MSX_F32: i64 ? Fn<cpu::F32, int64_t>::run(args...) : Fn<cpu::F32, int32_t>::run(args...); break;
  case MSX_F16: i64 ? Fn<cpu::F16, int64_t>::run(args...) : Fn<cpu::F16, int32_t>::run(args...); break;
  case MSX_BF16: i64 ? Fn<cpu::BF16, int64_t>::run(args...) : Fn<cpu::BF16, int32_t>::run(args...); break;
  case MSX_C64: i64 ? Fn<cpu::C64, int64_t>::run(args...) : Fn<cpu::C64, int32_t>::run(args...); break;
  }
}

template <class V, class I>
struct TransposeProductCpu {
  static void run(int64_t n_rows, int64_t n_cols, int64_t k, const void *data, const void *indices,
                  const void *indptr, const void *X, void *Y, int workers) {
    cpu::transpose_product<V, I>(n_rows, n_cols, k, data, indices, indptr, X, Y, workers);
  }
};

template <class V, class I>
struct TransposeCsrCpu {
  static void run(int64_t n_rows, int64_t n_cols, int64_t nnz, const void *data,
                  const void *indices, const void *indptr, void *t_data, void *t_indices,
                  void *t_indptr) {
    cpu::transpose_csr<V, I>(n_rows, n_cols, nnz, data, indices, indptr, t_data, t_indices,
                             t_indptr);
  }
};

template <class V, class I>
struct DataVjpCpu {
  static void run(int64_t n_rows, int64_t n_cols, int64_t k, bool single, const void *indices,
                  const void *indptr, const void *X, const void *cot, void *out, int workers) {
    cpu::data_vjp<V, I>(n_rows, n_cols, k, single, indices, indptr, X, cot, out, workers);
  }
};

int resolve_workers(int n_threads) { return n_threads > 0 ? n_threads : cpu::worker_count(); }

}  // namespace

extern "C" msx_status msx_csr_transpose_cpu(msx_vtype vt, msx_itype it, int64_t n_rows,
                                            int64_t n_cols, int64_t nnz, const void *data,
                                            const void *indices, const void *indptr, void *t_data,
                                            void *t_indices, void *t_indptr) {
  clear_error();
  msx_status st = check_cpu("csr_transpose", vt, it, n_rows, n_cols, nnz, data, indices, indptr);
  if (st != MSX_OK) return st;
  if (t_indptr == nullptr || (nnz > 0 && (t_data == nullptr || t_indices == nullptr)))
    return fail(MSX_EINVAL, "csr_transpose output buffers must be non-NULL.");
  return guarded("csr_transpose", [&] {
    dispatch_cpu<TransposeCsrCpu>(vt, it, n_rows, n_cols, nnz, data, indices, indptr, t_data,
                                  t_indices, t_indptr);
  });
}

extern "C" msx_status msx_csr_spmv_transpose_cpu(msx_vtype vt, msx_itype it, int64_t n_rows,
                                                 int64_t n_cols, int64_t nnz, const void *data,
                                                 const void *indices, const void *indptr,
                                                 const void *x, void *y, int n_threads) {
  clear_error();
  msx_status st = check_cpu("csr_matvec_transpose", vt, it, n_rows, n_cols, nnz, data, indices, indptr);
  if (st != MSX_OK) return st;
  if (n_cols > 0 && y == nullptr) return fail(MSX_EINVAL, "csr_matvec_transpose y is NULL.");
  if (n_rows > 0 && nnz > 0 && x == nullptr) return fail(MSX_EINVAL, "csr_matvec_transpose x is NULL.");
  const int workers = resolve_workers(n_threads);
  return guarded("csr_matvec_transpose", [&] {
    dispatch_cpu<TransposeProductCpu>(vt, it, n_rows, n_cols, int64_t{1}, data, indices, indptr, x,
                                      y, workers);
  });
}

extern "C" msx_status msx_csr_spmm_transpose_cpu(msx_vtype vt, msx_itype it, int64_t n_rows,
                                                 int64_t n_cols, int64_t nnz, const void *data,
                                                 const void *indices, const void *indptr, int64_t k,
                                                 const void *X, void *Y, int n_threads) {
  clear_error();
  msx_status st = check_cpu("csr_matmul_transpose", vt, it, n_rows, n_cols, nnz, data, indices, indptr);
  if (st != MSX_OK) return st;
  if (k < 0) return fail(MSX_EINVAL, "csr_matmul_transpose rhs column count must be non-negative.");
  if (n_cols > 0 && k > 0 && Y == nullptr) return fail(MSX_EINVAL, "csr_matmul_transpose Y is NULL.");
  if (n_rows > 0 && nnz > 0 && k > 0 && X == nullptr)
    return fail(MSX_EINVAL, "csr_matmul_transpose X is NULL.");
  const int workers = resolve_workers(n_threads);
  return guarded("csr_matmul_transpose", [&] {
    dispatch_cpu<TransposeProductCpu>(vt, it, n_rows, n_cols, k, data, indices, indptr, X, Y,
                                      workers);
  });
}

extern "C" msx_status msx_csr_spmv_data_vjp_cpu(msx_vtype vt, msx_itype it, int64_t n_rows,
                                                int64_t n_cols, int64_t nnz, const void *indices,
                                                const void *indptr, const void *x, const void *cot,
                                                void *out, int n_threads) {
  clear_error();
  msx_status st = check_cpu("csr_matvec_data_vjp", vt, it, n_rows, n_cols, nnz, indices, indices, indptr);
  if (st != MSX_OK) return st;
  if (nnz > 0 && (out == nullptr || cot == nullptr || (n_cols > 0 && x == nullptr)))
    return fail(MSX_EINVAL, "csr_matvec_data_vjp buffers must be non-NULL.");
  const int workers = resolve_workers(n_threads);
  return guarded("csr_matvec_data_vjp", [&] {
    dispatch_cpu<DataVjpCpu>(vt, it, n_rows, n_cols, int64_t{1}, true, indices, indptr, x, cot,
                             out, workers);
  });
}

extern "C" msx_status msx_csr_spmm_data_vjp_cpu(msx_vtype vt, msx_itype it, int64_t n_rows,
                                                int64_t n_cols, int64_t nnz, const void *indices,
                                                const void *indptr, int64_t k, const void *X,
                                                const void *cot, void *out, int n_threads) {
  clear_error();
  msx_status st = check_cpu("csr_matmul_data_vjp", vt, it, n_rows, n_cols, nnz, indices, indices, indptr);
  if (st != MSX_OK) return st;
  if (k < 0) return fail(MSX_EINVAL, "csr_matmul_data_vjp rhs column count must be non-negative.");
  if (nnz > 0 && (out == nullptr || (k > 0 && (cot == nullptr || (n_cols > 0 && X == nullptr)))))
    return fail(MSX_EINVAL, "csr_matmul_data_vjp buffers must be non-NULL.");
  const int workers = resolve_workers(n_threads);
  return guarded("csr_matmul_data_vjp", [&] {
    dispatch_cpu<DataVjpCpu>(vt, it, n_rows, n_cols, k, false, indices, indptr, X, cot, out,
                             workers);
  });
}
