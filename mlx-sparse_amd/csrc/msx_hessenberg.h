// msx_hessenberg.h - the small least-squares problem of restarted GMRES,
// solved on the host: min || H y - beta e1 || for an upper-Hessenberg H of
// (m + 1) x m (row-major, double), by one Givens rotation per column and a
// back substitution, with the reference's rank and finiteness tests
// (reference: src/linalg/common/common.h:143-234,
// least_squares_upper_hessenberg_givens_qr).  Shared by the device solver's
// host loop (csr_gmres.hip) and the CPU solver (csr_gmres_cpu.cpp).
#pragma once

#include <stdint.h>

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <vector>

namespace msx {

// y (m entries) from h ((m + 1) x m) and rhs (m + 1); false where the
// reference throws (a non-finite entry, a rank-deficient matrix, a
// degenerate rotation or diagonal, a non-finite solution).
inline bool hessenberg_least_squares(std::vector<double> h, std::vector<double> rhs, int64_t m,
                                     std::vector<double> &y) {
  const int64_t rows = m + 1, cols = m;
  if (m <= 0 || static_cast<int64_t>(h.size()) != rows * cols ||
      static_cast<int64_t>(rhs.size()) != rows)
    return false;
  double scale = 0.0;
  for (double v : h) {
    if (!std::isfinite(v)) return false;
    scale = std::max(scale, std::fabs(v));
  }
  for (double v : rhs)
    if (!std::isfinite(v)) return false;
  const double rank_tol = DBL_EPSILON * static_cast<double>(rows) * std::max(1.0, scale);
  if (scale <= rank_tol) return false;
  for (int64_t c = 0; c < cols; ++c) {
    const double top_c = h[c * cols + c], low_c = h[(c + 1) * cols + c];
    if (low_c == 0.0) continue;
    const double rad = std::hypot(top_c, low_c);
    if (!std::isfinite(rad) || rad <= rank_tol) return false;
    const double cs = top_c / rad, sn = low_c / rad;
    for (int64_t j = c; j < cols; ++j) {
      const double a = h[c * cols + j], b = h[(c + 1) * cols + j];
      h[c * cols + j] = cs * a + sn * b;
      h[(c + 1) * cols + j] = -sn * a + cs * b;
    }
    const double a = rhs[c], b = rhs[c + 1];
    rhs[c] = cs * a + sn * b;
    rhs[c + 1] = -sn * a + cs * b;
  }
  y.assign(static_cast<size_t>(cols), 0.0);
  for (int64_t i = cols - 1; i >= 0; --i) {
    double acc = rhs[i];
    for (int64_t j = i + 1; j < cols; ++j) acc -= h[i * cols + j] * y[j];
    const double d = h[i * cols + i];
    if (!std::isfinite(d) || std::fabs(d) <= rank_tol) return false;
    y[i] = acc / d;
    if (!std::isfinite(y[i])) return false;
  }
  return true;
}

}  // namespace msx
