// csr_adjoint.cpp - C++ primitive layer of the adjoint side.  Each function
// checks its operands with the reference op's messages, then calls the C ABI
// (device operands: the HIP entry point on ctx.stream; host operands: the
// native CPU entry point).
#include "sparse/csr_adjoint/csr_adjoint.h"

#include <stdexcept>
#include <string>

#include "common/validate.h"

namespace msx {
namespace {

void check_dims(int64_t n_rows, int64_t n_cols, const char *op) {
  if (n_rows < 0 || n_cols < 0)
    throw std::invalid_argument(std::string(op) + " shape dimensions must be non-negative.");
  if (n_rows >= 2147483647 || n_cols >= 2147483647)
    throw std::invalid_argument(std::string(op) + " shape dimensions must fit in int32.");
}

void check_csr(const ArrayView &data, const ArrayView &indices, const ArrayView &indptr,
               int64_t n_rows, const std::string &op) {
  require_rank(data, 1, (op + " data").c_str());
  require_rank(indices, 1, (op + " indices").c_str());
  require_rank(indptr, 1, (op + " indptr").c_str());
  require_supported_value_dtype(data, (op + " data").c_str());
  require_same_index_dtype(indices, indptr, (op + " indices").c_str(), (op + " indptr").c_str());
  require_size(indptr, n_rows + 1, (op + " indptr").c_str());
  if (indices.size() != data.size())
    throw std::invalid_argument(op + " data and indices must have equal length.");
}

void check_out(const ArrayView &out, const ArrayView &like, std::initializer_list<int64_t> shape,
               const std::string &op) {
  bool ok = out.ndim == static_cast<int>(shape.size()) && out.dtype == like.dtype;
  int i = 0;
  for (int64_t s : shape) ok = ok && out.shape[i++] == s;
  if (!ok) throw std::invalid_argument(op + " output buffer has the wrong shape or dtype.");
}

}  // namespace

void csr_transpose(const ArrayView &data, const ArrayView &indices, const ArrayView &indptr,
                   const ArrayView &out_data, const ArrayView &out_indices,
                   const ArrayView &out_indptr, int64_t n_rows, int64_t n_cols,
                   const ExecContext &ctx) {
  // reference: src/sparse/csr_transpose/csr_transpose.cpp, csr_transpose
  check_dims(n_rows, n_cols, "csr_transpose");
  check_csr(data, indices, indptr, n_rows, "csr_transpose");
  require_same_device({&data, &indices, &indptr, &out_data, &out_indices, &out_indptr},
                      "csr_transpose");
  check_out(out_data, data, {data.size()}, "csr_transpose");
  check_out(out_indices, indices, {indices.size()}, "csr_transpose");
  check_out(out_indptr, indptr, {n_cols + 1}, "csr_transpose");
  for (const ArrayView *a : {&data, &indices, &indptr, &out_data, &out_indices, &out_indptr})
    require_contiguous(*a, "csr_transpose operand");
  const msx_vtype vt = to_vtype(data.dtype);
  const msx_itype it = to_itype(indices.dtype);
  if (data.device >= 0)
    check_status(msx_csr_transpose(vt, it, n_rows, n_cols, data.size(), data.ptr, indices.ptr,
                                   indptr.ptr, out_data.ptr, out_indices.ptr, out_indptr.ptr,
                                   ctx.stream),
                 "csr_transpose");
  else
    check_status(msx_csr_transpose_cpu(vt, it, n_rows, n_cols, data.size(), data.ptr, indices.ptr,
                                       indptr.ptr, out_data.ptr, out_indices.ptr, out_indptr.ptr),
                 "csr_transpose");
}

void csr_matvec_transpose(const ArrayView &data, const ArrayView &indices,
                          const ArrayView &indptr, const ArrayView &x, const ArrayView &out,
                          int64_t n_rows, int64_t n_cols, const ExecContext &ctx) {
  // reference: src/sparse/csr_matvec_transpose/csr_matvec_transpose.cpp,
  // csr_matvec_transpose
  const std::string op = "csr_matvec_transpose";
  check_dims(n_rows, n_cols, op.c_str());
  check_csr(data, indices, indptr, n_rows, op);
  require_rank(x, 1, "csr_matvec_transpose x");
  require_same_value_dtype(data, x, "csr_matvec_transpose data", "csr_matvec_transpose x");
  require_size(x, n_rows, "csr_matvec_transpose x");
  require_same_device({&data, &indices, &indptr, &x, &out}, op.c_str());
  check_out(out, data, {n_cols}, op);
  for (const ArrayView *a : {&data, &indices, &indptr, &x, &out})
    require_contiguous(*a, "csr_matvec_transpose operand");
  const msx_vtype vt = to_vtype(data.dtype);
  const msx_itype it = to_itype(indices.dtype);
  if (data.device >= 0)
    check_status(msx_csr_spmv_transpose(vt, it, n_rows, n_cols, data.size(), data.ptr,
                                        indices.ptr, indptr.ptr, x.ptr, out.ptr, ctx.stream),
                 op.c_str());
  else
    check_status(msx_csr_spmv_transpose_cpu(vt, it, n_rows, n_cols, data.size(), data.ptr,
                                            indices.ptr, indptr.ptr, x.ptr, out.ptr, ctx.n_threads),
                 op.c_str());
}

void csr_matmul_transpose(const ArrayView &data, const ArrayView &indices,
                          const ArrayView &indptr, const ArrayView &rhs, const ArrayView &out,
                          int64_t n_rows, int64_t n_cols, const ExecContext &ctx) {
  // reference: src/sparse/csr_matmul_transpose/csr_matmul_transpose.cpp,
  // csr_matmul_transpose
  const std::string op = "csr_matmul_transpose";
  check_dims(n_rows, n_cols, op.c_str());
  check_csr(data, indices, indptr, n_rows, op);
  require_rank(rhs, 2, "csr_matmul_transpose rhs");
  require_same_value_dtype(data, rhs, "csr_matmul_transpose data", "csr_matmul_transpose rhs");
  if (rhs.shape[0] != n_rows)
    throw std::invalid_argument(
        "csr_matmul_transpose rhs first dimension must equal the sparse matrix row count.");
  const int64_t k = rhs.shape[1];
  require_same_device({&data, &indices, &indptr, &rhs, &out}, op.c_str());
  check_out(out, data, {n_cols, k}, op);
  for (const ArrayView *a : {&data, &indices, &indptr, &rhs, &out})
    require_contiguous(*a, "csr_matmul_transpose operand");
  const msx_vtype vt = to_vtype(data.dtype);
  const msx_itype it = to_itype(indices.dtype);
  if (data.device >= 0)
    check_status(msx_csr_spmm_transpose(vt, it, n_rows, n_cols, data.size(), data.ptr,
                                        indices.ptr, indptr.ptr, k, rhs.ptr, k, out.ptr, k,
                                        ctx.stream),
                 op.c_str());
  else
    check_status(msx_csr_spmm_transpose_cpu(vt, it, n_rows, n_cols, data.size(), data.ptr,
                                            indices.ptr, indptr.ptr, k, rhs.ptr, out.ptr,
                                            ctx.n_threads),
                 op.c_str());
}

void csr_matvec_data_vjp(const ArrayView &indices, const ArrayView &indptr, const ArrayView &x,
                         const ArrayView &cotangent, const ArrayView &out, int64_t n_rows,
                         int64_t n_cols, const ExecContext &ctx, const msx_csr_plan *plan) {
  // reference: src/sparse/csr_matvec_data_vjp/csr_matvec_data_vjp.cpp,
  // csr_matvec_data_vjp
  const char *op = "csr_matvec_data_vjp";
  check_dims(n_rows, n_cols, op);
  require_rank(indices, 1, "csr_matvec_data_vjp indices");
  require_rank(indptr, 1, "csr_matvec_data_vjp indptr");
  require_rank(x, 1, "csr_matvec_data_vjp x");
  require_rank(cotangent, 1, "csr_matvec_data_vjp cotangent");
  require_supported_value_dtype(x, "csr_matvec_data_vjp x");
  require_same_value_dtype(x, cotangent, "csr_matvec_data_vjp x", "csr_matvec_data_vjp cotangent");
  require_same_index_dtype(indices, indptr, "csr_matvec_data_vjp indices",
                           "csr_matvec_data_vjp indptr");
  require_size(indptr, n_rows + 1, "csr_matvec_data_vjp indptr");
  require_size(x, n_cols, "csr_matvec_data_vjp x");
  require_size(cotangent, n_rows, "csr_matvec_data_vjp cotangent");
  require_same_device({&indices, &indptr, &x, &cotangent, &out}, op);
  check_out(out, x, {indices.size()}, op);
  for (const ArrayView *a : {&indices, &indptr, &x, &cotangent, &out})
    require_contiguous(*a, "csr_matvec_data_vjp operand");
  const msx_vtype vt = to_vtype(x.dtype);
  const msx_itype it = to_itype(indices.dtype);
  if (x.device >= 0)
    check_status(msx_csr_spmv_data_vjp(vt, it, n_rows, n_cols, indices.size(), indices.ptr,
                                       indptr.ptr, x.ptr, cotangent.ptr, out.ptr, plan,
                                       ctx.stream),
                 op);
  else
    check_status(msx_csr_spmv_data_vjp_cpu(vt, it, n_rows, n_cols, indices.size(), indices.ptr,
                                           indptr.ptr, x.ptr, cotangent.ptr, out.ptr,
                                           ctx.n_threads),
                 op);
}

void csr_matmul_data_vjp(const ArrayView &indices, const ArrayView &indptr, const ArrayView &rhs,
                         const ArrayView &cotangent, const ArrayView &out, int64_t n_rows,
                         int64_t n_cols, const ExecContext &ctx) {
  // reference: src/sparse/csr_matmul_data_vjp/csr_matmul_data_vjp.cpp,
  // csr_matmul_data_vjp
  const char *op = "csr_matmul_data_vjp";
  check_dims(n_rows, n_cols, op);
  require_rank(indices, 1, "csr_matmul_data_vjp indices");
  require_rank(indptr, 1, "csr_matmul_data_vjp indptr");
  require_rank(rhs, 2, "csr_matmul_data_vjp rhs");
  require_rank(cotangent, 2, "csr_matmul_data_vjp cotangent");
  require_supported_value_dtype(rhs, "csr_matmul_data_vjp rhs");
  require_same_value_dtype(rhs, cotangent, "csr_matmul_data_vjp rhs",
                           "csr_matmul_data_vjp cotangent");
  require_same_index_dtype(indices, indptr, "csr_matmul_data_vjp indices",
                           "csr_matmul_data_vjp indptr");
  require_size(indptr, n_rows + 1, "csr_matmul_data_vjp indptr");
  if (rhs.shape[0] != n_cols)
    throw std::invalid_argument(
        "csr_matmul_data_vjp rhs first dimension must equal the sparse matrix column count.");
  if (cotangent.shape[0] != n_rows)
    throw std::invalid_argument(
        "csr_matmul_data_vjp cotangent first dimension must equal the sparse matrix row count.");
  if (rhs.shape[1] != cotangent.shape[1])
    throw std::invalid_argument(
        "csr_matmul_data_vjp rhs and cotangent must have the same number of columns.");
  const int64_t k = rhs.shape[1];
  require_same_device({&indices, &indptr, &rhs, &cotangent, &out}, op);
  check_out(out, rhs, {indices.size()}, op);
  for (const ArrayView *a : {&indices, &indptr, &rhs, &cotangent, &out})
    require_contiguous(*a, "csr_matmul_data_vjp operand");
  const msx_vtype vt = to_vtype(rhs.dtype);
  const msx_itype it = to_itype(indices.dtype);
  if (rhs.device >= 0)
    check_status(msx_csr_spmm_data_vjp(vt, it, n_rows, n_cols, indices.size(), indices.ptr,
                                       indptr.ptr, k, rhs.ptr, k, cotangent.ptr, k, out.ptr,
                                       ctx.stream),
                 op);
  else
    check_status(msx_csr_spmm_data_vjp_cpu(vt, it, n_rows, n_cols, indices.size(), indices.ptr,
                                           indptr.ptr, k, rhs.ptr, cotangent.ptr, out.ptr,
                                           ctx.n_threads),
                 op);
}

}  // namespace msx
