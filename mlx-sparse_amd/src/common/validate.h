// validate.h - argument validators of the C++ primitive layer.
//
// Same checks and texts as the reference's validators (reference:
// src/common/common.cpp:104-177); they throw std::invalid_argument, which
// the binding surfaces as ValueError.
#pragma once

#include <sstream>
#include <stdexcept>
#include <string>

#include "common/array_view.h"
#include "msx_sparse.h"

namespace msx {

inline bool is_value_dtype(DType d) {
  return d == DType::Float32 || d == DType::Float16 || d == DType::BFloat16 ||
         d == DType::Complex64;
}

inline void require_rank(const ArrayView &a, int ndim, const char *name) {
  if (a.ndim != ndim) {
    std::ostringstream msg;
    msg << name << " must be rank-" << ndim << ", got rank " << a.ndim << ".";
    throw std::invalid_argument(msg.str());
  }
}

inline void require_supported_value_dtype(const ArrayView &a, const char *name) {
  if (!is_value_dtype(a.dtype)) {
    std::ostringstream msg;
    msg << name << " must have dtype float32, float16, bfloat16, or complex64, got "
        << a.dtype_name << ".";
    throw std::invalid_argument(msg.str());
  }
}

inline void require_index_dtype(const ArrayView &a, const char *name) {
  if (a.dtype != DType::Int32 && a.dtype != DType::Int64) {
    std::ostringstream msg;
    msg << name << " must have dtype int32 or int64, got " << a.dtype_name << ".";
    throw std::invalid_argument(msg.str());
  }
}

inline void require_same_value_dtype(const ArrayView &l, const ArrayView &r, const char *ln,
                                     const char *rn) {
  require_supported_value_dtype(l, ln);
  require_supported_value_dtype(r, rn);
  if (l.dtype != r.dtype) {
    std::ostringstream msg;
    msg << ln << " and " << rn << " must have the same dtype, got " << l.dtype_name << " and "
        << r.dtype_name << ".";
    throw std::invalid_argument(msg.str());
  }
}

inline void require_same_index_dtype(const ArrayView &l, const ArrayView &r, const char *ln,
                                     const char *rn) {
  require_index_dtype(l, ln);
  require_index_dtype(r, rn);
  if (l.dtype != r.dtype) {
    std::ostringstream msg;
    msg << ln << " and " << rn << " must have the same dtype, got " << l.dtype_name << " and "
        << r.dtype_name << ".";
    throw std::invalid_argument(msg.str());
  }
}

inline void require_size(const ArrayView &a, int64_t expected, const char *name) {
  if (a.size() != expected) {
    std::ostringstream msg;
    msg << name << " must have size " << expected << ", got " << a.size() << ".";
    throw std::invalid_argument(msg.str());
  }
}

// All arrays of one call live in one memory space (new: the reference's MLX
// arrays are in unified memory).
inline void require_same_device(std::initializer_list<const ArrayView *> arrays, const char *op) {
  const ArrayView *first = *arrays.begin();
  for (const ArrayView *a : arrays) {
    if (a->device != first->device) {
      std::ostringstream msg;
      msg << op << " inputs must be on one device, got "
          << (first->device < 0 ? std::string("cpu") : "gpu:" + std::to_string(first->device))
          << " and " << (a->device < 0 ? std::string("cpu") : "gpu:" + std::to_string(a->device))
          << ".";
      throw std::invalid_argument(msg.str());
    }
  }
}

inline void require_contiguous(const ArrayView &a, const char *name) {
  if (!a.contiguous()) throw std::invalid_argument(std::string(name) + " must be contiguous.");
}

inline msx_vtype to_vtype(DType d) {
  switch (d) {
  case DType::Float32: return MSX_F32;
  case DType::Float16: return MSX_F16;
  case DType::BFloat16: return MSX_BF16;
  case DType::Complex64: return MSX_C64;
  default: break;
  }
  throw std::runtime_error("unsupported value dtype.");
}

inline msx_itype to_itype(DType d) { return d == DType::Int64 ? MSX_I64 : MSX_I32; }

// Status of a C-ABI call -> exception of the matching Python class.
[[noreturn]] void throw_status(msx_status st, const char *op);

inline void check_status(msx_status st, const char *op) {
  if (st != MSX_OK) throw_status(st, op);
}

}  // namespace msx
