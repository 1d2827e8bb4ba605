// array_view.h - framework-neutral description of a strided array, the input
// of the C++ primitive layer.  The binding fills it from torch tensors; the
// layer itself never sees a framework type.
#pragma once

#include <stdint.h>

#include <string>

namespace msx {

enum class DType { Float32, Float16, BFloat16, Complex64, Int32, Int64, Other };

struct ArrayView {
  void *ptr = nullptr;
  DType dtype = DType::Other;
  std::string dtype_name;  // framework spelling, for error texts
  int ndim = 0;                     // the layer handles ranks 0..3
  int64_t shape[3] = {0, 0, 0};
  int64_t strides[3] = {1, 1, 1};  // in elements
  int device = -1;                 // -1: host memory; >= 0: HIP device ordinal

  int64_t size() const {
    int64_t s = 1;
    for (int i = 0; i < ndim && i < 3; ++i) s *= shape[i];
    return ndim == 0 ? 1 : s;
  }
  bool contiguous() const {
    int64_t expect = 1;
    for (int i = ndim - 1; i >= 0; --i) {
      if (shape[i] > 1 && strides[i] != expect) return false;
      expect *= shape[i];
    }
    return true;
  }
};

// Where and how a primitive runs.
struct ExecContext {
  void *stream = nullptr;  // hipStream_t for device arrays
  int n_threads = 0;       // host worker count (0: resolve from the environment)
};

}  // namespace msx
