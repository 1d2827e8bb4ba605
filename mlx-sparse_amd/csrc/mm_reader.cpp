// mm_reader.cpp - Matrix Market ingestion: the text files of the SuiteSparse
// collection (reference fixtures tests/fixtures/suitesparse/HB/*.mtx, read by
// the reference's tests with scipy.io.mmread and turned into CSRArray by
// from_scipy, mlx_sparse/_construct.py:854-975).
//
// Host code, multithreaded: the data section is split into chunks at line
// boundaries, each thread counts then parses its chunk (std::from_chars,
// correctly rounded), symmetric kinds are expanded, entries are bucketed by
// row in file order (counting sort), each row is sorted by column and
// duplicates are summed in double in file order, then every value is
// rounded once to the storage type.  The output is canonical CSR, as
// from_scipy(canonical=True) builds it.
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <cctype>
#include <charconv>
#include <cmath>
#include <cstdio>
#include <string>
#include <thread>
#include <vector>

#include "msx_sparse.h"

namespace msx {
msx_status fail(msx_status code, const std::string &msg);
void clear_error();
}  // namespace msx

namespace {

enum Format { kCoordinate = 0, kArray = 1 };
enum Field { kReal = 0, kInteger = 1, kComplex = 2, kPattern = 3 };
enum Symmetry { kGeneral = 0, kSymmetric = 1, kSkew = 2, kHermitian = 3 };

struct File {
  std::string text;
  size_t data_begin = 0;  // first byte after the size line
  msx_mm_info info{};
};

std::string lower(std::string s) {
  for (char &c : s) c = static_cast<char>(std::tolower(static_cast<unsigned char>(c)));
  return s;
}

bool read_all(const char *path, std::string &out) {
  FILE *f = std::fopen(path, "rb");
  if (!f) return false;
  std::fseek(f, 0, SEEK_END);
  const long size = std::ftell(f);
  std::fseek(f, 0, SEEK_SET);
  if (size < 0) {
    std::fclose(f);
    return false;
  }
  out.resize(static_cast<size_t>(size));
  const size_t got = size > 0 ? std::fread(&out[0], 1, static_cast<size_t>(size), f) : 0;
  std::fclose(f);
  return got == static_cast<size_t>(size);
}

const char *skip_space(const char *p, const char *end) {
  while (p < end && (*p == ' ' || *p == '\t' || *p == '\r')) ++p;
  return p;
}

template <class T>
bool parse_num(const char *&p, const char *end, T &v) {
  p = skip_space(p, end);
  if (p < end && *p == '+') ++p;  // from_chars takes no leading '+'
  auto r = std::from_chars(p, end, v);
  if (r.ec != std::errc()) return false;
  p = r.ptr;
  return true;
}

// Header and size line.
msx_status open_file(const char *path, File &f) {
  if (!read_all(path, f.text))
    return msx::fail(MSX_EINVAL, std::string("mmread: cannot read '") + path + "'.");
  const std::string &t = f.text;
  const size_t eol = t.find('\n');
  std::string head = lower(t.substr(0, eol == std::string::npos ? t.size() : eol));
  char tag[64] = {0}, obj[64] = {0}, fmt[64] = {0}, fld[64] = {0}, sym[64] = {0};
  if (std::sscanf(head.c_str(), "%63s %63s %63s %63s %63s", tag, obj, fmt, fld, sym) != 5 ||
      std::string(tag) != "%%matrixmarket" || std::string(obj) != "matrix")
    return msx::fail(MSX_EINVAL, "mmread: not a Matrix Market matrix file (bad header line).");
  msx_mm_info &in = f.info;
  const std::string sf(fmt), sd(fld), ss(sym);
  if (sf == "coordinate") in.format = kCoordinate;
  else if (sf == "array") in.format = kArray;
  else return msx::fail(MSX_EINVAL, "mmread: unknown format '" + sf + "'.");
  if (sd == "real" || sd == "double") in.field = kReal;
  else if (sd == "integer") in.field = kInteger;
  else if (sd == "complex") in.field = kComplex;
  else if (sd == "pattern") in.field = kPattern;
  else return msx::fail(MSX_EINVAL, "mmread: unknown field '" + sd + "'.");
  if (ss == "general") in.symmetry = kGeneral;
  else if (ss == "symmetric") in.symmetry = kSymmetric;
  else if (ss == "skew-symmetric") in.symmetry = kSkew;
  else if (ss == "hermitian") in.symmetry = kHermitian;
  else return msx::fail(MSX_EINVAL, "mmread: unknown symmetry '" + ss + "'.");
  if (in.format == kArray && in.field == kPattern)
    return msx::fail(MSX_EINVAL, "mmread: a pattern matrix must use the coordinate format.");
  // size line: the first line after the header that is neither a comment nor blank
  size_t pos = eol == std::string::npos ? t.size() : eol + 1;
  while (pos < t.size()) {
    size_t e = t.find('\n', pos);
    if (e == std::string::npos) e = t.size();
    const char *p = skip_space(t.data() + pos, t.data() + e);
    if (p < t.data() + e && *p != '%') {
      int64_t a = 0, b = 0, c = 0;
      const char *end = t.data() + e;
      if (!parse_num(p, end, a) || !parse_num(p, end, b))
        return msx::fail(MSX_EINVAL, "mmread: bad size line.");
      if (in.format == kCoordinate && !parse_num(p, end, c))
        return msx::fail(MSX_EINVAL, "mmread: bad size line (rows, columns, entries).");
      if (a < 0 || b < 0 || c < 0) return msx::fail(MSX_EINVAL, "mmread: negative size.");
      if (in.symmetry != kGeneral && a != b)
        return msx::fail(MSX_EINVAL, "mmread: a symmetric matrix must be square.");
      in.n_rows = a;
      in.n_cols = b;
      if (in.format == kArray) {
        // symmetric arrays store the lower triangle (skew: without the diagonal)
        const int64_t n = a;
        in.entries = in.symmetry == kGeneral ? a * b
                     : in.symmetry == kSkew  ? n * (n - 1) / 2
                                             : n * (n + 1) / 2;
        in.nnz_bound = a * b;
      } else {
        in.entries = c;
        in.nnz_bound = in.symmetry == kGeneral ? c : 2 * c;
      }
      f.data_begin = e < t.size() ? e + 1 : t.size();
      return MSX_OK;
    }
    pos = e + 1;
  }
  return msx::fail(MSX_EINVAL, "mmread: missing size line.");
}

// Data lines of [begin, end): calls fn(line_begin, line_end) for each
// non-blank, non-comment line.
template <class Fn>
void for_lines(const char *begin, const char *end, Fn fn) {
  const char *p = begin;
  while (p < end) {
    const char *e = static_cast<const char *>(memchr(p, '\n', static_cast<size_t>(end - p)));
    if (!e) e = end;
    const char *q = skip_space(p, e);
    if (q < e && *q != '%') fn(q, e);
    p = e + 1;
  }
}

struct Chunks {
  std::vector<const char *> begin, end;
  std::vector<int64_t> offset;  // first entry index of each chunk
};

Chunks split(const File &f, int threads) {
  Chunks c;
  const char *b = f.text.data() + f.data_begin;
  const char *e = f.text.data() + f.text.size();
  const size_t size = static_cast<size_t>(e - b);
  const int parts = std::max(1, std::min<int>(threads, static_cast<int>(size / (1 << 16)) + 1));
  const char *cur = b;
  for (int i = 0; i < parts; ++i) {
    const char *stop = i == parts - 1 ? e : b + size * (i + 1) / parts;
    if (stop < cur) stop = cur;
    if (stop < e) {
      const char *nl = static_cast<const char *>(memchr(stop, '\n', static_cast<size_t>(e - stop)));
      stop = nl ? nl + 1 : e;
    }
    c.begin.push_back(cur);
    c.end.push_back(stop);
    cur = stop;
  }
  c.offset.assign(c.begin.size() + 1, 0);
  return c;
}

template <class Fn>
void run_parallel(int parts, Fn fn) {
  if (parts <= 1) {
    fn(0);
    return;
  }
  std::vector<std::thread> pool;
  for (int i = 0; i < parts; ++i) pool.emplace_back(fn, i);
  for (auto &t : pool) t.join();
}

int resolve_threads(int n_threads) {
  if (n_threads > 0) return n_threads;
  const int w = msx_cpu_worker_count();
  return w > 0 ? w : 1;
}

// Entries of the data section: 0-based (row, col) and value (re, im).
struct Entries {
  std::vector<int64_t> row, col;
  std::vector<double> re, im;
};

msx_status parse_entries(const File &f, int threads, Entries &out) {
  const msx_mm_info &in = f.info;
  Chunks c = split(f, threads);
  const int parts = static_cast<int>(c.begin.size());
  std::vector<int64_t> counts(parts, 0);
  run_parallel(parts, [&](int i) {
    int64_t k = 0;
    for_lines(c.begin[i], c.end[i], [&](const char *, const char *) { ++k; });
    counts[i] = k;
  });
  for (int i = 0; i < parts; ++i) c.offset[i + 1] = c.offset[i] + counts[i];
  const int64_t total = c.offset[parts];
  if (total != in.entries)
    return msx::fail(MSX_EINVAL, "mmread: the file holds " + std::to_string(total) +
                                     " data lines, the size line promises " +
                                     std::to_string(in.entries) + ".");
  const bool cplx = in.field == kComplex;
  out.row.resize(total);
  out.col.resize(total);
  out.re.resize(total);
  if (cplx) out.im.resize(total);
  std::vector<int> bad(parts, 0);
  std::vector<int64_t> bad_line(parts, 0);
  run_parallel(parts, [&](int i) {
    int64_t k = c.offset[i];
    for_lines(c.begin[i], c.end[i], [&](const char *p, const char *e) {
      if (bad[i]) return;
      int64_t r = 0, cc = 0;
      double re = 1.0, im = 0.0;
      bool ok = true;
      if (in.format == kCoordinate) {
        ok = parse_num(p, e, r) && parse_num(p, e, cc);
        r -= 1;
        cc -= 1;
        if (ok && (r < 0 || r >= in.n_rows || cc < 0 || cc >= in.n_cols)) ok = false;
      } else {
        // array: column-major, lower triangle for symmetric kinds
        int64_t idx = k, col = 0, row = 0;
        if (in.symmetry == kGeneral) {
          col = in.n_rows > 0 ? idx / in.n_rows : 0;
          row = idx - col * in.n_rows;
        } else {
          const int64_t n = in.n_rows;
          const int64_t skip = in.symmetry == kSkew ? 1 : 0;
          col = 0;
          while (col < n && idx >= n - col - skip) {
            idx -= n - col - skip;
            ++col;
          }
          row = col + skip + idx;
        }
        r = row;
        cc = col;
      }
      if (ok && in.field != kPattern) {
        if (in.field == kInteger) {
          int64_t iv = 0;
          ok = parse_num(p, e, iv);
          re = static_cast<double>(iv);
        } else {
          ok = parse_num(p, e, re);
        }
        if (ok && cplx) ok = parse_num(p, e, im);
      }
      if (!ok) {
        bad[i] = 1;
        bad_line[i] = k;
        return;
      }
      out.row[k] = r;
      out.col[k] = cc;
      out.re[k] = re;
      if (cplx) out.im[k] = im;
      ++k;
    });
  });
  for (int i = 0; i < parts; ++i)
    if (bad[i])
      return msx::fail(MSX_EINVAL, "mmread: bad data line (entry " +
                                       std::to_string(bad_line[i] + 1) + ").");
  return MSX_OK;
}

// Storage rounding, once, from double.
uint16_t half_from_double(double v) {
  uint64_t b;
  memcpy(&b, &v, 8);
  const uint16_t sign = static_cast<uint16_t>((b >> 48) & 0x8000u);
  const int exp = static_cast<int>((b >> 52) & 0x7ff);
  uint64_t man = b & ((uint64_t{1} << 52) - 1);
  if (exp == 0x7ff) return static_cast<uint16_t>(sign | 0x7c00u | (man ? 0x200u : 0u));
  const int e = exp - 1023;  // unbiased
  if (e > 15) return static_cast<uint16_t>(sign | 0x7c00u);
  // value = 1.man * 2^e (normal doubles); half normals need e >= -14
  uint64_t full = (exp == 0 ? man : (man | (uint64_t{1} << 52)));
  int shift;  // bits to drop from `full` (53 significant bits) for the half's 10/11 bits
  uint16_t hexp;
  if (e >= -14) {
    shift = 52 - 10;
    hexp = static_cast<uint16_t>(e + 15);
  } else {
    shift = 52 - 10 + (-14 - e);  // subnormal half
    hexp = 0;
    if (exp == 0 || shift > 63) return sign;  // far below the smallest half
  }
  uint64_t kept = full >> shift;
  const uint64_t rem = full & ((uint64_t{1} << shift) - 1);
  const uint64_t halfway = uint64_t{1} << (shift - 1);
  if (rem > halfway || (rem == halfway && (kept & 1))) ++kept;
  uint32_t out;
  if (hexp == 0) {
    out = static_cast<uint32_t>(kept);  // may round up into the first normal (0x400)
  } else {
    // kept includes the implicit bit at 1 << 10; a carry to 1 << 11 bumps the exponent
    uint32_t ex = hexp;
    if (kept >> 11) {
      kept >>= 1;
      ++ex;
    }
    if (ex >= 31) return static_cast<uint16_t>(sign | 0x7c00u);
    out = (ex << 10) | static_cast<uint32_t>(kept & 0x3ffu);
  }
  return static_cast<uint16_t>(sign | out);
}

uint16_t bf16_from_float(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  const uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return static_cast<uint16_t>(u >> 16);
}

void store(msx_vtype vt, void *data, int64_t k, double re, double im) {
  switch (vt) {
  case MSX_F32: static_cast<float *>(data)[k] = static_cast<float>(re); break;
  case MSX_F16: static_cast<uint16_t *>(data)[k] = half_from_double(re); break;
  case MSX_BF16:
    // the reference's from_scipy reaches bfloat16 through float32
    static_cast<uint16_t *>(data)[k] = bf16_from_float(static_cast<float>(re));
    break;
  case MSX_C64:
    static_cast<float *>(data)[2 * k] = static_cast<float>(re);
    static_cast<float *>(data)[2 * k + 1] = static_cast<float>(im);
    break;
  }
}

template <class I>
msx_status build_csr(const msx_mm_info &in, const Entries &en, msx_vtype vt, int64_t capacity,
                     void *data, void *indices_v, void *indptr_v, int64_t *nnz_out, int threads) {
  auto *indices = static_cast<I *>(indices_v);
  auto *indptr = static_cast<I *>(indptr_v);
  const int64_t n_rows = in.n_rows;
  const int64_t m = static_cast<int64_t>(en.row.size());
  const bool cplx = in.field == kComplex;
  // expanded entry list: (row, col, k, mirrored)
  const bool sym = in.symmetry != kGeneral;
  std::vector<int64_t> count(n_rows + 1, 0);
  for (int64_t k = 0; k < m; ++k) {
    count[en.row[k] + 1]++;
    if (sym && en.row[k] != en.col[k]) count[en.col[k] + 1]++;
  }
  for (int64_t r = 0; r < n_rows; ++r) count[r + 1] += count[r];
  const int64_t total = count[n_rows];
  // slots in file order; each slot remembers its source entry (negative: mirrored)
  std::vector<int64_t> next(count.begin(), count.end() - 1);
  std::vector<int64_t> src(total), col(total);
  for (int64_t k = 0; k < m; ++k) {
    const int64_t s = next[en.row[k]]++;
    src[s] = k;
    col[s] = en.col[k];
    if (sym && en.row[k] != en.col[k]) {
      const int64_t t = next[en.col[k]]++;
      src[t] = -(k + 1);
      col[t] = en.row[k];
    }
  }
  // per row: stable sort by column, sum duplicates (double, in order)
  std::vector<int64_t> row_nnz(n_rows, 0);
  const int parts = std::max(1, std::min<int>(threads, static_cast<int>(n_rows / 4096) + 1));
  run_parallel(parts, [&](int t) {
    std::vector<std::pair<int64_t, int64_t>> tmp;
    for (int64_t r = n_rows * t / parts; r < n_rows * (t + 1) / parts; ++r) {
      const int64_t b = count[r], e = count[r + 1];
      tmp.clear();
      for (int64_t s = b; s < e; ++s) tmp.emplace_back(col[s], src[s]);
      std::stable_sort(tmp.begin(), tmp.end(),
                       [](const auto &a, const auto &c) { return a.first < c.first; });
      int64_t kept = 0;
      for (size_t i = 0; i < tmp.size(); ++i)
        if (i == 0 || tmp[i].first != tmp[i - 1].first) ++kept;
      row_nnz[r] = kept;
      for (int64_t s = b; s < e; ++s) {
        col[s] = tmp[s - b].first;
        src[s] = tmp[s - b].second;
      }
    }
  });
  int64_t nnz = 0;
  for (int64_t r = 0; r < n_rows; ++r) nnz += row_nnz[r];
  *nnz_out = nnz;
  if (nnz > capacity)
    return msx::fail(MSX_EINVAL, "mmread: " + std::to_string(nnz) +
                                     " stored values exceed the buffers' capacity " +
                                     std::to_string(capacity) + ".");
  if (sizeof(I) == 4 && nnz > 2147483647)
    return msx::fail(MSX_EINVAL, "mmread: too many values for int32 indices.");
  std::vector<int64_t> out_ptr(n_rows + 1, 0);
  for (int64_t r = 0; r < n_rows; ++r) out_ptr[r + 1] = out_ptr[r] + row_nnz[r];
  for (int64_t r = 0; r <= n_rows; ++r) indptr[r] = static_cast<I>(out_ptr[r]);
  run_parallel(parts, [&](int t) {
    for (int64_t r = n_rows * t / parts; r < n_rows * (t + 1) / parts; ++r) {
      int64_t o = out_ptr[r] - 1;
      int64_t last = -1;
      double sre = 0.0, sim = 0.0;
      for (int64_t s = count[r]; s < count[r + 1]; ++s) {
        const int64_t k = src[s] >= 0 ? src[s] : -src[s] - 1;
        double re = en.re[k], im = cplx ? en.im[k] : 0.0;
        if (src[s] < 0) {  // mirrored entry
          if (in.symmetry == kSkew) {
            re = -re;
            im = -im;
          } else if (in.symmetry == kHermitian) {
            im = -im;
          }
        }
        if (col[s] != last) {
          if (o >= out_ptr[r]) store(vt, data, o, sre, sim);
          ++o;
          indices[o] = static_cast<I>(col[s]);
          last = col[s];
          sre = re;
          sim = im;
        } else {
          sre += re;
          sim += im;
        }
      }
      if (o >= out_ptr[r]) store(vt, data, o, sre, sim);
    }
  });
  return MSX_OK;
}

}  // namespace

extern "C" msx_status msx_mm_info_read(const char *path, msx_mm_info *info) {
  msx::clear_error();
  if (path == nullptr || info == nullptr) return msx::fail(MSX_EINVAL, "mmread: NULL argument.");
  File f;
  const msx_status st = open_file(path, f);
  if (st != MSX_OK) return st;
  *info = f.info;
  return MSX_OK;
}

extern "C" msx_status msx_mm_read_csr(const char *path, msx_vtype vt, msx_itype it,
                                      int64_t capacity, void *data, void *indices, void *indptr,
                                      int64_t *nnz, int n_threads) {
  msx::clear_error();
  if (path == nullptr || nnz == nullptr || indptr == nullptr)
    return msx::fail(MSX_EINVAL, "mmread: NULL argument.");
  if (vt != MSX_F32 && vt != MSX_F16 && vt != MSX_BF16 && vt != MSX_C64)
    return msx::fail(MSX_ETYPE, "mmread: unsupported value dtype.");
  if (it != MSX_I32 && it != MSX_I64)
    return msx::fail(MSX_ETYPE, "mmread: indices must be int32 or int64.");
  if (capacity > 0 && (data == nullptr || indices == nullptr))
    return msx::fail(MSX_EINVAL, "mmread: NULL output buffer.");
  try {
    File f;
    msx_status st = open_file(path, f);
    if (st != MSX_OK) return st;
    if (f.info.field == kComplex && vt != MSX_C64)
      return msx::fail(MSX_ETYPE, "mmread: a complex matrix needs complex64 values.");
    if (it == MSX_I32 && (f.info.n_rows >= 2147483647 || f.info.n_cols >= 2147483647))
      return msx::fail(MSX_EINVAL, "mmread: dimensions do not fit int32 indices.");
    Entries en;
    st = parse_entries(f, resolve_threads(n_threads), en);
    if (st != MSX_OK) return st;
    return it == MSX_I32
               ? build_csr<int32_t>(f.info, en, vt, capacity, data, indices, indptr, nnz,
                                    resolve_threads(n_threads))
               : build_csr<int64_t>(f.info, en, vt, capacity, data, indices, indptr, nnz,
                                    resolve_threads(n_threads));
  } catch (const std::bad_alloc &) {
    return msx::fail(MSX_ENOMEM, "mmread: out of host memory.");
  }
}

extern "C" msx_status msx_mm_read_dense(const char *path, msx_vtype vt, int64_t capacity,
                                        void *out, int n_threads) {
  msx::clear_error();
  if (path == nullptr) return msx::fail(MSX_EINVAL, "mmread: NULL argument.");
  if (vt != MSX_F32 && vt != MSX_F16 && vt != MSX_BF16 && vt != MSX_C64)
    return msx::fail(MSX_ETYPE, "mmread: unsupported value dtype.");
  try {
    File f;
    msx_status st = open_file(path, f);
    if (st != MSX_OK) return st;
    if (f.info.field == kComplex && vt != MSX_C64)
      return msx::fail(MSX_ETYPE, "mmread: a complex matrix needs complex64 values.");
    const int64_t n_rows = f.info.n_rows, n_cols = f.info.n_cols;
    if (n_rows * n_cols > capacity)
      return msx::fail(MSX_EINVAL, "mmread: the dense output buffer is too small.");
    if (n_rows * n_cols > 0 && out == nullptr)
      return msx::fail(MSX_EINVAL, "mmread: NULL output buffer.");
    Entries en;
    st = parse_entries(f, resolve_threads(n_threads), en);
    if (st != MSX_OK) return st;
    // dense row-major: zeros, then entries (duplicates summed), then mirrors
    const bool cplx = f.info.field == kComplex;
    std::vector<double> re(static_cast<size_t>(n_rows * n_cols), 0.0), im;
    if (cplx) im.assign(re.size(), 0.0);
    for (size_t k = 0; k < en.row.size(); ++k) {
      const int64_t r = en.row[k], c = en.col[k];
      const double vr = en.re[k], vi = cplx ? en.im[k] : 0.0;
      re[r * n_cols + c] += vr;
      if (cplx) im[r * n_cols + c] += vi;
      if (f.info.symmetry != kGeneral && r != c) {
        const double sgn = f.info.symmetry == kSkew ? -1.0 : 1.0;
        re[c * n_cols + r] += sgn * vr;
        if (cplx) im[c * n_cols + r] += f.info.symmetry == kHermitian ? -vi : sgn * vi;
      }
    }
    for (int64_t i = 0; i < n_rows * n_cols; ++i) store(vt, out, i, re[i], cplx ? im[i] : 0.0);
    return MSX_OK;
  } catch (const std::bad_alloc &) {
    return msx::fail(MSX_ENOMEM, "mmread: out of host memory.");
  }
}
