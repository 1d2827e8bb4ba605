// capi.hip - extern "C" entry points of libmsx_sparse: argument checks, error
// state and dispatch to the HIP launchers.
//
// The checks mirror the reference op constructors (reference:
// src/sparse/csr_matvec/csr_matvec.cpp:326-356,
// src/sparse/csr_matmul/csr_matmul.cpp:383-418) on raw sizes: shape
// dimensions non-negative and representable as int, sizes consistent, and
// pointers present wherever a non-empty buffer is read or written.
#include <hip/hip_runtime.h>

#include <string>

#include "msx_internal.h"
#include "msx_sparse.h"

namespace msx {
namespace {
thread_local std::string g_last_error;
constexpr int64_t kIntMax = 2147483647;
}  // namespace

void set_error(const std::string &msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

msx_status fail(msx_status code, const std::string &msg) {
  g_last_error = msg;
  return code;
}

msx_status hip_fail(hipError_t err, const char *what) {
  g_last_error = std::string(what) + ": " + hipGetErrorName(err) + " (" + hipGetErrorString(err) + ")";
  return MSX_EHIP;
}

size_t value_bytes(msx_vtype vt) {
  switch (vt) {
  case MSX_F32: return 4;
  case MSX_F16: return 2;
  case MSX_BF16: return 2;
  case MSX_C64: return 8;
  }
  return 0;
}

size_t index_bytes(msx_itype it) { return it == MSX_I64 ? 8 : 4; }
bool valid_vtype(int vt) { return vt >= MSX_F32 && vt <= MSX_C64; }
bool valid_itype(int it) { return it == MSX_I32 || it == MSX_I64; }

namespace {

msx_status check_common(const char *op, msx_vtype vt, msx_itype it, int64_t n_rows, int64_t n_cols,
                        int64_t nnz, const void *data, const void *indices, const void *indptr) {
  if (!valid_itype(it)) return fail(MSX_ETYPE, std::string(op) + " requires int32 or int64 indices.");
  if (!valid_vtype(vt)) return fail(MSX_ETYPE, std::string(op) + " unsupported value dtype.");
  if (n_rows < 0 || n_cols < 0 || nnz < 0)
    return fail(MSX_EINVAL, std::string(op) + " shape dimensions must be non-negative.");
  if (n_rows >= kIntMax || n_cols > kIntMax)
    return fail(MSX_EINVAL, std::string(op) + " shape dimensions must fit in int32.");
  if (indptr == nullptr) return fail(MSX_EINVAL, std::string(op) + " indptr is NULL.");
  if (nnz > 0 && (data == nullptr || indices == nullptr))
    return fail(MSX_EINVAL, std::string(op) + " data and indices must be non-NULL when nnz > 0.");
  return MSX_OK;
}

}  // namespace

msx_status check_plan(const char *op, const msx_csr_plan *plan, msx_vtype vt, msx_itype it,
                      int64_t n_rows, int64_t n_cols, int64_t nnz, const void *data,
                      const void *indices, const void *indptr) {
  if (plan == nullptr) return MSX_OK;
  if (plan->itype != it || plan->n_rows != n_rows || plan->nnz != nnz)
    return fail(MSX_EINVAL, std::string(op) + ": plan was built for a different matrix.");
  // The row blocks come from one indptr buffer: another buffer (even of the
  // same length and nnz) may hold other rows.
  if (plan->indptr != indptr)
    return fail(MSX_EINVAL, std::string(op) + ": plan was built from another indptr buffer.");
  if (plan->bound && (plan->bound_data != data || plan->bound_indices != indices ||
                      plan->vtype != vt || plan->n_cols != n_cols))
    return fail(MSX_EINVAL, std::string(op) + ": plan is bound to other data/indices buffers.");
  int dev = -1;
  MSX_HIP_TRY(hipGetDevice(&dev));
  if (dev != plan->device)
    return fail(MSX_EINVAL, std::string(op) + ": plan lives on another device.");
  return MSX_OK;
}

}  // namespace msx

using namespace msx;

extern "C" int msx_abi_version(void) { return MSX_ABI_VERSION; }

extern "C" const char *msx_last_error(void) { return g_last_error.c_str(); }

extern "C" msx_status msx_device_count(int *count) {
  clear_error();
  if (count == nullptr) return fail(MSX_EINVAL, "msx_device_count: count is NULL.");
  int c = 0;
  hipError_t e = hipGetDeviceCount(&c);
  if (e == hipErrorNoDevice) {
    (void)hipGetLastError();
    c = 0;
  } else if (e != hipSuccess) {
    *count = 0;
    return hip_fail(e, "hipGetDeviceCount");
  }
  *count = c;
  return MSX_OK;
}

extern "C" msx_status msx_csr_spmv(msx_vtype vt, msx_itype it, int64_t n_rows, int64_t n_cols,
                                   int64_t nnz, const void *data, const void *indices,
                                   const void *indptr, const void *x, void *y,
                                   const msx_csr_plan *plan, void *stream) {
  clear_error();
  msx_status st = check_common("csr_matvec", vt, it, n_rows, n_cols, nnz, data, indices, indptr);
  if (st != MSX_OK) return st;
  if (n_rows > 0 && y == nullptr) return fail(MSX_EINVAL, "csr_matvec y is NULL.");
  if (n_cols > 0 && nnz > 0 && x == nullptr) return fail(MSX_EINVAL, "csr_matvec x is NULL.");
  st = check_plan("csr_matvec", plan, vt, it, n_rows, n_cols, nnz, data, indices, indptr);
  if (st != MSX_OK) return st;
  if (n_rows == 0) return MSX_OK;
  return launch_spmv(vt, it, n_rows, n_cols, nnz, data, indices, indptr, x, y, plan,
                     static_cast<hipStream_t>(stream));
}

extern "C" msx_status msx_csr_spmm(msx_vtype vt, msx_itype it, int64_t n_rows, int64_t n_cols,
                                   int64_t nnz, const void *data, const void *indices,
                                   const void *indptr, int64_t k, const void *X, int64_t ldx,
                                   void *Y, int64_t ldy, const msx_csr_plan *plan, void *stream) {
  clear_error();
  msx_status st = check_common("csr_matmul", vt, it, n_rows, n_cols, nnz, data, indices, indptr);
  if (st != MSX_OK) return st;
  if (k < 0 || k > kIntMax) return fail(MSX_EINVAL, "csr_matmul rhs column count must fit in int32.");
  if (ldx < k || ldy < k)
    return fail(MSX_EINVAL, "csr_matmul leading dimensions must be at least the column count.");
  if (n_rows > 0 && k > 0 && Y == nullptr) return fail(MSX_EINVAL, "csr_matmul Y is NULL.");
  if (n_cols > 0 && k > 0 && nnz > 0 && X == nullptr)
    return fail(MSX_EINVAL, "csr_matmul X is NULL.");
  st = check_plan("csr_matmul", plan, vt, it, n_rows, n_cols, nnz, data, indices, indptr);
  if (st != MSX_OK) return st;
  if (n_rows == 0 || k == 0) return MSX_OK;
  return launch_spmm(vt, it, n_rows, n_cols, nnz, data, indices, indptr, k, X, ldx, Y, ldy, plan,
                     static_cast<hipStream_t>(stream));
}
