// bindings.cpp - the `mlx_sparse._ext` Python module (pybind11).
//
// Mirrors the reference nanobind module's entry points for this path
// (reference: src/bindings.cpp:279-295 `_compiled_capabilities`,
// :874-883 `csr_matvec`, :905-915 `csr_batched_matvec`, :965-975
// `csr_matmul`, :998-1008 `csr_batched_matmul`, :661-665 `csr_transpose`,
// :942-947 `csr_matvec_transpose`, :1035-1040 `csr_matmul_transpose`; the
// value gradients, internal to the reference's VJPs, are bound as
// `csr_matvec_data_vjp` / `csr_matmul_data_vjp`; the solvers, :1470-1482
// `csr_gmres` among them): same names and argument
// order (data, indices, indptr, x | rhs, n_rows, n_cols).  Arrays are torch
// tensors; the module reads their pointer, dtype, shape, strides and device
// through the tensor's Python attributes, so no torch headers are compiled
// here.  Inputs are made contiguous (the reference's mx::contiguous), the
// output is allocated with torch.empty on the inputs' device, device work is
// ordered on torch's current stream for that device, and errors surface as
// ValueError (std::invalid_argument), RuntimeError or MemoryError.
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <memory>
#include <string>
#include <vector>

#include "common/array_view.h"
#include "common/validate.h"
#include "msx_sparse.h"
#include "linalg/csr_cg.h"
#include "linalg/csr_krylov.h"
#include "sparse/csr_adjoint/csr_adjoint.h"
#include "sparse/csr_batched_matmul/csr_batched_matmul.h"
#include "sparse/csr_batched_matvec/csr_batched_matvec.h"
#include "sparse/csr_matmul/csr_matmul.h"
#include "sparse/csr_matvec/csr_matvec.h"

namespace py = pybind11;
using msx::ArrayView;
using msx::DType;

namespace {

py::module_ &torch() {
  static py::module_ mod = py::module_::import("torch");
  return mod;
}

DType dtype_of(const std::string &name) {
  if (name == "float32") return DType::Float32;
  if (name == "float16") return DType::Float16;
  if (name == "bfloat16") return DType::BFloat16;
  if (name == "complex64") return DType::Complex64;
  if (name == "int32") return DType::Int32;
  if (name == "int64") return DType::Int64;
  return DType::Other;
}

std::string dtype_name(py::handle dtype) {
  std::string s = py::str(dtype);
  const std::string prefix = "torch.";
  if (s.rfind(prefix, 0) == 0) s = s.substr(prefix.size());
  return s;
}

int device_index(py::handle tensor) {
  py::object dev = tensor.attr("device");
  const std::string type = py::str(dev.attr("type"));
  if (type == "cpu") return -1;
  if (type != "cuda") throw std::invalid_argument("mlx_sparse supports cpu and HIP (cuda) tensors only, got " + type + ".");
  py::object idx = dev.attr("index");
  return idx.is_none() ? torch().attr("cuda").attr("current_device")().cast<int>() : idx.cast<int>();
}

ArrayView view_of(py::handle t) {
  ArrayView v;
  v.dtype_name = dtype_name(t.attr("dtype"));
  v.dtype = dtype_of(v.dtype_name);
  v.ndim = t.attr("dim")().cast<int>();
  if (v.ndim <= 3) {
    auto shape = t.attr("shape").cast<std::vector<int64_t>>();
    auto strides = t.attr("stride")().cast<std::vector<int64_t>>();
    for (int i = 0; i < v.ndim; ++i) {
      v.shape[i] = shape[i];
      v.strides[i] = strides[i];
    }
  }
  v.ptr = reinterpret_cast<void *>(t.attr("data_ptr")().cast<uintptr_t>());
  v.device = device_index(t);
  return v;
}

py::object as_tensor(py::handle obj) {
  if (py::isinstance(obj, torch().attr("Tensor"))) return py::reinterpret_borrow<py::object>(obj);
  return torch().attr("as_tensor")(obj);
}

py::object contiguous(py::handle obj) { return as_tensor(obj).attr("contiguous")(); }

void *stream_for(int device) {
  if (device < 0) return nullptr;
  const int current = torch().attr("cuda").attr("current_device")().cast<int>();
  if (current != device)
    throw std::invalid_argument("mlx_sparse: GPU operands must be on the current device (cuda:" +
                                std::to_string(current) + "), got cuda:" + std::to_string(device) + ".");
  py::object s = torch().attr("cuda").attr("current_stream")(device);
  return reinterpret_cast<void *>(s.attr("cuda_stream").cast<uintptr_t>());
}

// Owner of a device plan; destroyed with the Python object.
struct Plan {
  msx_csr_plan *p = nullptr;
  int64_t n_rows = 0;
  int64_t nnz = 0;
  std::string index_dtype;
  int device = -1;
  py::object bound;  // tensors a bound plan was built from (kept alive)
  ~Plan() {
    if (p) msx_csr_plan_destroy(p);
  }
};

std::shared_ptr<Plan> make_plan(py::handle indptr_obj, int64_t n_rows, int64_t nnz,
                                int64_t block_nnz, py::object data_obj, py::object indices_obj,
                                int64_t n_cols, int slice_mode) {
  py::object indptr = contiguous(indptr_obj);
  ArrayView v = view_of(indptr);
  msx::require_rank(v, 1, "csr_plan indptr");
  msx::require_index_dtype(v, "csr_plan indptr");
  msx::require_size(v, n_rows + 1, "csr_plan indptr");
  if (v.device < 0) throw std::invalid_argument("csr_plan indptr must be a GPU tensor.");
  void *stream = stream_for(v.device);
  auto plan = std::make_shared<Plan>();
  plan->n_rows = n_rows;
  plan->nnz = nnz;
  plan->index_dtype = v.dtype_name;
  plan->device = v.device;
  msx_status st;
  if (data_obj.is_none()) {
    py::gil_scoped_release nogil;
    st = msx_csr_plan_create(msx::to_itype(v.dtype), n_rows, nnz, v.ptr, block_nnz, stream,
                             &plan->p);
  } else {
    // A bound plan reads the values it was built from: the caller keeps these
    // exact (contiguous, same-device) tensors alive and unchanged.
    const ArrayView vd = view_of(data_obj), vi = view_of(indices_obj);
    msx::require_rank(vd, 1, "csr_plan data");
    msx::require_rank(vi, 1, "csr_plan indices");
    msx::require_supported_value_dtype(vd, "csr_plan data");
    msx::require_same_index_dtype(vi, v, "csr_plan indices", "csr_plan indptr");
    msx::require_size(vd, nnz, "csr_plan data");
    msx::require_size(vi, nnz, "csr_plan indices");
    msx::require_same_device({&vd, &vi, &v}, "csr_plan");
    msx::require_contiguous(vd, "csr_plan data");
    msx::require_contiguous(vi, "csr_plan indices");
    plan->bound = py::make_tuple(data_obj, indices_obj, indptr);
    msx_plan_options opts{block_nnz, slice_mode, 0};
    py::gil_scoped_release nogil;
    st = msx_csr_plan_create_bound(msx::to_vtype(vd.dtype), msx::to_itype(v.dtype), n_rows, n_cols,
                                   nnz, vd.ptr, vi.ptr, v.ptr, &opts, stream, &plan->p);
  }
  msx::check_status(st, "csr_plan");
  return plan;
}

// The matrix's values changed (indices and indptr did not): rewrite the
// bound plan's copies from `data` and keep `data` alive in its place.
void plan_refresh(Plan &plan, py::handle data_obj) {
  if (plan.bound.is_none()) return;  // row blocks hold no values
  py::tuple bound = plan.bound.cast<py::tuple>();
  const ArrayView vd = view_of(data_obj), vi = view_of(bound[1]);
  msx::require_rank(vd, 1, "csr_plan_refresh data");
  msx::require_same_value_dtype(vd, view_of(bound[0]), "csr_plan_refresh data", "plan data");
  msx::require_size(vd, plan.nnz, "csr_plan_refresh data");
  msx::require_same_device({&vd, &vi}, "csr_plan_refresh");
  msx::require_contiguous(vd, "csr_plan_refresh data");
  void *stream = stream_for(vd.device);
  msx_status st;
  {
    py::gil_scoped_release nogil;
    st = msx_csr_plan_refresh(plan.p, vd.ptr, stream);
  }
  msx::check_status(st, "csr_plan_refresh");
  plan.bound = py::make_tuple(py::reinterpret_borrow<py::object>(data_obj), bound[1], bound[2]);
}

const msx_csr_plan *plan_ptr(const py::object &plan) {
  if (plan.is_none()) return nullptr;
  return plan.cast<std::shared_ptr<Plan>>()->p;
}

py::object empty_like_out(const ArrayView &data, py::handle data_obj, py::tuple shape) {
  py::dict kw;
  kw["dtype"] = data_obj.attr("dtype");
  kw["device"] = data_obj.attr("device");
  return torch().attr("empty")(shape, **kw);
}

py::object csr_matvec(py::handle data_o, py::handle indices_o, py::handle indptr_o, py::handle x_o,
                      int64_t n_rows, int64_t n_cols, py::object plan, int n_threads) {
  py::object data = contiguous(data_o), indices = contiguous(indices_o),
             indptr = contiguous(indptr_o), x = contiguous(x_o);
  const ArrayView vd = view_of(data), vi = view_of(indices), vp = view_of(indptr), vx = view_of(x);
  py::object out = empty_like_out(vd, data, py::make_tuple(std::max<int64_t>(n_rows, 0)));
  const ArrayView vo = view_of(out);
  msx::ExecContext ctx;
  ctx.n_threads = n_threads;
  ctx.stream = vd.device >= 0 ? stream_for(vd.device) : nullptr;
  const msx_csr_plan *p = plan_ptr(plan);
  if (vd.device >= 0) {
    msx::csr_matvec(vd, vi, vp, vx, vo, n_rows, n_cols, p, ctx);
  } else {
    py::gil_scoped_release nogil;
    msx::csr_matvec(vd, vi, vp, vx, vo, n_rows, n_cols, nullptr, ctx);
  }
  return out;
}

py::object csr_matmul(py::handle data_o, py::handle indices_o, py::handle indptr_o,
                      py::handle rhs_o, int64_t n_rows, int64_t n_cols, py::object plan,
                      int n_threads) {
  py::object data = contiguous(data_o), indices = contiguous(indices_o),
             indptr = contiguous(indptr_o), rhs = contiguous(rhs_o);
  const ArrayView vd = view_of(data), vi = view_of(indices), vp = view_of(indptr),
                  vr = view_of(rhs);
  if (vr.ndim != 2) msx::require_rank(vr, 2, "csr_matmul rhs");
  py::object out = empty_like_out(vd, data, py::make_tuple(std::max<int64_t>(n_rows, 0), vr.shape[1]));
  const ArrayView vo = view_of(out);
  msx::ExecContext ctx;
  ctx.n_threads = n_threads;
  ctx.stream = vd.device >= 0 ? stream_for(vd.device) : nullptr;
  const msx_csr_plan *p = plan_ptr(plan);
  if (vd.device >= 0) {
    msx::csr_matmul(vd, vi, vp, vr, vo, n_rows, n_cols, p, ctx);
  } else {
    py::gil_scoped_release nogil;
    msx::csr_matmul(vd, vi, vp, vr, vo, n_rows, n_cols, nullptr, ctx);
  }
  return out;
}

py::object csr_batched_matvec(py::handle data_o, py::handle indices_o, py::handle indptr_o,
                              py::handle rhs_o, int64_t n_rows, int64_t n_cols, int n_threads) {
  py::object data = contiguous(data_o), indices = contiguous(indices_o),
             indptr = contiguous(indptr_o), rhs = contiguous(rhs_o);
  const ArrayView vd = view_of(data), vi = view_of(indices), vp = view_of(indptr),
                  vr = view_of(rhs);
  if (vr.ndim != 2) msx::require_rank(vr, 2, "csr_batched_matvec rhs");
  py::object out = empty_like_out(vd, data, py::make_tuple(vr.shape[0], std::max<int64_t>(n_rows, 0)));
  const ArrayView vo = view_of(out);
  msx::ExecContext ctx;
  ctx.n_threads = n_threads;
  ctx.stream = vd.device >= 0 ? stream_for(vd.device) : nullptr;
  if (vd.device >= 0) {
    msx::csr_batched_matvec(vd, vi, vp, vr, vo, n_rows, n_cols, ctx);
  } else {
    py::gil_scoped_release nogil;
    msx::csr_batched_matvec(vd, vi, vp, vr, vo, n_rows, n_cols, ctx);
  }
  return out;
}

py::object csr_batched_matmul(py::handle data_o, py::handle indices_o, py::handle indptr_o,
                              py::handle rhs_o, int64_t n_rows, int64_t n_cols, int n_threads) {
  py::object data = contiguous(data_o), indices = contiguous(indices_o),
             indptr = contiguous(indptr_o), rhs = contiguous(rhs_o);
  const ArrayView vd = view_of(data), vi = view_of(indices), vp = view_of(indptr),
                  vr = view_of(rhs);
  if (vr.ndim != 3) msx::require_rank(vr, 3, "csr_batched_matmul rhs");
  py::object out = empty_like_out(
      vd, data, py::make_tuple(vr.shape[0], std::max<int64_t>(n_rows, 0), vr.shape[2]));
  const ArrayView vo = view_of(out);
  msx::ExecContext ctx;
  ctx.n_threads = n_threads;
  ctx.stream = vd.device >= 0 ? stream_for(vd.device) : nullptr;
  if (vd.device >= 0) {
    msx::csr_batched_matmul(vd, vi, vp, vr, vo, n_rows, n_cols, ctx);
  } else {
    py::gil_scoped_release nogil;
    msx::csr_batched_matmul(vd, vi, vp, vr, vo, n_rows, n_cols, ctx);
  }
  return out;
}

msx::ExecContext context_for(const ArrayView &v, int n_threads) {
  msx::ExecContext ctx;
  ctx.n_threads = n_threads;
  ctx.stream = v.device >= 0 ? stream_for(v.device) : nullptr;
  return ctx;
}

py::tuple csr_transpose(py::handle data_o, py::handle indices_o, py::handle indptr_o,
                        int64_t n_rows, int64_t n_cols) {
  py::object data = contiguous(data_o), indices = contiguous(indices_o),
             indptr = contiguous(indptr_o);
  const ArrayView vd = view_of(data), vi = view_of(indices), vp = view_of(indptr);
  if (vd.ndim != 1) msx::require_rank(vd, 1, "csr_transpose data");
  if (vi.ndim != 1) msx::require_rank(vi, 1, "csr_transpose indices");
  py::object od = empty_like_out(vd, data, py::make_tuple(vd.shape[0]));
  py::object oi = empty_like_out(vi, indices, py::make_tuple(vi.shape[0]));
  py::object op = empty_like_out(vp, indptr, py::make_tuple(std::max<int64_t>(n_cols, 0) + 1));
  const ArrayView vod = view_of(od), voi = view_of(oi), vop = view_of(op);
  const msx::ExecContext ctx = context_for(vd, 0);
  if (vd.device >= 0) {
    msx::csr_transpose(vd, vi, vp, vod, voi, vop, n_rows, n_cols, ctx);
  } else {
    py::gil_scoped_release nogil;
    msx::csr_transpose(vd, vi, vp, vod, voi, vop, n_rows, n_cols, ctx);
  }
  return py::make_tuple(od, oi, op);
}

// (t_pos, t_indices, t_indptr): the transpose's structure and, per entry,
// the position of A it holds (GPU operands).
py::tuple csr_transpose_positions(py::handle indices_o, py::handle indptr_o, int64_t n_rows,
                                  int64_t n_cols) {
  py::object indices = contiguous(indices_o), indptr = contiguous(indptr_o);
  const ArrayView vi = view_of(indices), vp = view_of(indptr);
  if (vi.ndim != 1) msx::require_rank(vi, 1, "csr_transpose_positions indices");
  msx::require_same_index_dtype(vi, vp, "csr_transpose_positions indices",
                                "csr_transpose_positions indptr");
  msx::require_size(vp, n_rows + 1, "csr_transpose_positions indptr");
  msx::require_same_device({&vi, &vp}, "csr_transpose_positions");
  if (vi.device < 0) throw std::invalid_argument("csr_transpose_positions needs GPU tensors.");
  py::dict kw;
  kw["dtype"] = torch().attr("int32");
  kw["device"] = indices.attr("device");
  py::object pos = torch().attr("empty")(py::make_tuple(vi.shape[0]), **kw);
  py::object oi = empty_like_out(vi, indices, py::make_tuple(vi.shape[0]));
  py::object op = empty_like_out(vp, indptr, py::make_tuple(std::max<int64_t>(n_cols, 0) + 1));
  const ArrayView vpos = view_of(pos), voi = view_of(oi), vop = view_of(op);
  void *stream = stream_for(vi.device);
  msx_status st;
  {
    py::gil_scoped_release nogil;
    st = msx_csr_transpose_positions(msx::to_itype(vi.dtype), n_rows, n_cols, vi.shape[0], vi.ptr,
                                     vp.ptr, static_cast<int32_t *>(vpos.ptr), voi.ptr, vop.ptr,
                                     stream);
  }
  msx::check_status(st, "csr_transpose_positions");
  return py::make_tuple(pos, oi, op);
}

// out[i] = data[t_pos[i]] (conjugated on request), in place (GPU operands).
void csr_transpose_values(py::handle data_o, py::handle pos_o, bool conjugate, py::handle out_o) {
  py::object data = contiguous(data_o), pos = contiguous(pos_o);
  const ArrayView vd = view_of(data), vpos = view_of(pos), vo = view_of(out_o);
  msx::require_rank(vd, 1, "csr_transpose_values data");
  msx::require_same_value_dtype(vd, vo, "csr_transpose_values data", "csr_transpose_values out");
  if (vpos.dtype != DType::Int32) throw std::invalid_argument("csr_transpose_values positions must be int32.");
  msx::require_size(vpos, vd.shape[0], "csr_transpose_values positions");
  msx::require_size(vo, vd.shape[0], "csr_transpose_values out");
  msx::require_contiguous(vo, "csr_transpose_values out");
  msx::require_same_device({&vd, &vpos, &vo}, "csr_transpose_values");
  if (vd.device < 0) throw std::invalid_argument("csr_transpose_values needs GPU tensors.");
  void *stream = stream_for(vd.device);
  msx_status st;
  {
    py::gil_scoped_release nogil;
    st = msx_csr_transpose_values(msx::to_vtype(vd.dtype), vd.shape[0], vd.ptr,
                                  static_cast<const int32_t *>(vpos.ptr), conjugate ? 1 : 0,
                                  vo.ptr, stream);
  }
  msx::check_status(st, "csr_transpose_values");
}

// (slot1 int16, src1 int32, slot2 int16): the layout of the two-pass
// regather of values of `like`'s dtype, from the transpose positions.
py::tuple csr_transpose_layout(py::handle pos_o, py::handle like_o) {
  py::object pos = contiguous(pos_o);
  const ArrayView vpos = view_of(pos), vl = view_of(like_o);
  msx::require_rank(vpos, 1, "csr_transpose_layout positions");
  if (vpos.dtype != DType::Int32) throw std::invalid_argument("csr_transpose_layout positions must be int32.");
  if (vpos.device < 0) throw std::invalid_argument("csr_transpose_layout needs GPU tensors.");
  const int64_t n = vpos.shape[0];
  py::dict k16, k32;
  k16["dtype"] = torch().attr("int16");
  k16["device"] = pos.attr("device");
  k32["dtype"] = torch().attr("int32");
  k32["device"] = pos.attr("device");
  py::object slot1 = torch().attr("empty")(py::make_tuple(n), **k16);
  py::object src1 = torch().attr("empty")(py::make_tuple(n), **k32);
  py::object slot2 = torch().attr("empty")(py::make_tuple(n), **k16);
  const ArrayView v1 = view_of(slot1), vs = view_of(src1), v2 = view_of(slot2);
  void *stream = stream_for(vpos.device);
  msx_status st;
  {
    py::gil_scoped_release nogil;
    st = msx_csr_transpose_layout(msx::to_vtype(vl.dtype), n, static_cast<const int32_t *>(vpos.ptr),
                                  static_cast<uint16_t *>(v1.ptr), static_cast<uint32_t *>(vs.ptr),
                                  static_cast<uint16_t *>(v2.ptr), stream);
  }
  msx::check_status(st, "csr_transpose_layout");
  return py::make_tuple(slot1, src1, slot2);
}

// out = data regathered through a layout of csr_transpose_layout; scratch:
// as many values as data (overwritten).
void csr_transpose_values_layout(py::handle data_o, py::handle slot1_o, py::handle src1_o,
                                 py::handle slot2_o, bool conjugate, py::handle scratch_o,
                                 py::handle out_o) {
  py::object data = contiguous(data_o), slot1 = contiguous(slot1_o), src1 = contiguous(src1_o),
             slot2 = contiguous(slot2_o);
  const ArrayView vd = view_of(data), v1 = view_of(slot1), vs = view_of(src1), v2 = view_of(slot2),
                  vsc = view_of(scratch_o), vo = view_of(out_o);
  const char *op = "csr_transpose_values_layout";
  msx::require_rank(vd, 1, "csr_transpose_values_layout data");
  msx::require_same_value_dtype(vd, vo, "csr_transpose_values_layout data",
                                "csr_transpose_values_layout out");
  msx::require_same_value_dtype(vd, vsc, "csr_transpose_values_layout data",
                                "csr_transpose_values_layout scratch");
  if (v1.dtype_name != "int16" || v2.dtype_name != "int16" || vs.dtype != DType::Int32)
    throw std::invalid_argument("csr_transpose_values_layout layout must be (int16, int32, int16).");
  for (const ArrayView *v : {&v1, &vs, &v2, &vsc, &vo})
    msx::require_size(*v, vd.shape[0], "csr_transpose_values_layout operand");
  msx::require_contiguous(vsc, "csr_transpose_values_layout scratch");
  msx::require_contiguous(vo, "csr_transpose_values_layout out");
  msx::require_same_device({&vd, &v1, &vs, &v2, &vsc, &vo}, op);
  if (vd.device < 0) throw std::invalid_argument("csr_transpose_values_layout needs GPU tensors.");
  void *stream = stream_for(vd.device);
  msx_status st;
  {
    py::gil_scoped_release nogil;
    st = msx_csr_transpose_values_layout(
        msx::to_vtype(vd.dtype), vd.shape[0], vd.ptr, static_cast<const uint16_t *>(v1.ptr),
        static_cast<const uint32_t *>(vs.ptr), static_cast<const uint16_t *>(v2.ptr),
        conjugate ? 1 : 0, vsc.ptr, vo.ptr, stream);
  }
  msx::check_status(st, op);
}

py::object csr_matvec_transpose(py::handle data_o, py::handle indices_o, py::handle indptr_o,
                                py::handle x_o, int64_t n_rows, int64_t n_cols, int n_threads) {
  py::object data = contiguous(data_o), indices = contiguous(indices_o),
             indptr = contiguous(indptr_o), x = contiguous(x_o);
  const ArrayView vd = view_of(data), vi = view_of(indices), vp = view_of(indptr), vx = view_of(x);
  py::object out = empty_like_out(vd, data, py::make_tuple(std::max<int64_t>(n_cols, 0)));
  const ArrayView vo = view_of(out);
  const msx::ExecContext ctx = context_for(vd, n_threads);
  if (vd.device >= 0) {
    msx::csr_matvec_transpose(vd, vi, vp, vx, vo, n_rows, n_cols, ctx);
  } else {
    py::gil_scoped_release nogil;
    msx::csr_matvec_transpose(vd, vi, vp, vx, vo, n_rows, n_cols, ctx);
  }
  return out;
}

py::object csr_matmul_transpose(py::handle data_o, py::handle indices_o, py::handle indptr_o,
                                py::handle rhs_o, int64_t n_rows, int64_t n_cols, int n_threads) {
  py::object data = contiguous(data_o), indices = contiguous(indices_o),
             indptr = contiguous(indptr_o), rhs = contiguous(rhs_o);
  const ArrayView vd = view_of(data), vi = view_of(indices), vp = view_of(indptr),
                  vr = view_of(rhs);
  if (vr.ndim != 2) msx::require_rank(vr, 2, "csr_matmul_transpose rhs");
  py::object out =
      empty_like_out(vd, data, py::make_tuple(std::max<int64_t>(n_cols, 0), vr.shape[1]));
  const ArrayView vo = view_of(out);
  const msx::ExecContext ctx = context_for(vd, n_threads);
  if (vd.device >= 0) {
    msx::csr_matmul_transpose(vd, vi, vp, vr, vo, n_rows, n_cols, ctx);
  } else {
    py::gil_scoped_release nogil;
    msx::csr_matmul_transpose(vd, vi, vp, vr, vo, n_rows, n_cols, ctx);
  }
  return out;
}

py::object csr_matvec_data_vjp(py::handle indices_o, py::handle indptr_o, py::handle x_o,
                               py::handle cot_o, int64_t n_rows, int64_t n_cols, int n_threads,
                               const py::object &plan) {
  py::object indices = contiguous(indices_o), indptr = contiguous(indptr_o), x = contiguous(x_o),
             cot = contiguous(cot_o);
  const ArrayView vi = view_of(indices), vp = view_of(indptr), vx = view_of(x), vc = view_of(cot);
  if (vi.ndim != 1) msx::require_rank(vi, 1, "csr_matvec_data_vjp indices");
  py::object out = empty_like_out(vx, x, py::make_tuple(vi.shape[0]));
  const ArrayView vo = view_of(out);
  const msx::ExecContext ctx = context_for(vx, n_threads);
  if (vx.device >= 0) {
    msx::csr_matvec_data_vjp(vi, vp, vx, vc, vo, n_rows, n_cols, ctx, plan_ptr(plan));
  } else {
    py::gil_scoped_release nogil;
    msx::csr_matvec_data_vjp(vi, vp, vx, vc, vo, n_rows, n_cols, ctx);
  }
  return out;
}

py::object csr_matmul_data_vjp(py::handle indices_o, py::handle indptr_o, py::handle rhs_o,
                               py::handle cot_o, int64_t n_rows, int64_t n_cols, int n_threads) {
  py::object indices = contiguous(indices_o), indptr = contiguous(indptr_o),
             rhs = contiguous(rhs_o), cot = contiguous(cot_o);
  const ArrayView vi = view_of(indices), vp = view_of(indptr), vr = view_of(rhs),
                  vc = view_of(cot);
  if (vi.ndim != 1) msx::require_rank(vi, 1, "csr_matmul_data_vjp indices");
  py::object out = empty_like_out(vr, rhs, py::make_tuple(vi.shape[0]));
  const ArrayView vo = view_of(out);
  const msx::ExecContext ctx = context_for(vr, n_threads);
  if (vr.device >= 0) {
    msx::csr_matmul_data_vjp(vi, vp, vr, vc, vo, n_rows, n_cols, ctx);
  } else {
    py::gil_scoped_release nogil;
    msx::csr_matmul_data_vjp(vi, vp, vr, vc, vo, n_rows, n_cols, ctx);
  }
  return out;
}

py::tuple solve_cg(py::handle data_o, py::handle indices_o, py::handle indptr_o, py::handle b_o,
                   py::handle x0_o, py::object inv_diag_o, int64_t n_rows, int64_t n_cols,
                   float rtol, float atol, int64_t maxiter, py::object plan) {
  py::object data = contiguous(data_o), indices = contiguous(indices_o),
             indptr = contiguous(indptr_o), b = contiguous(b_o), x0 = contiguous(x0_o);
  const ArrayView vd = view_of(data), vi = view_of(indices), vp = view_of(indptr), vb = view_of(b),
                  vx0 = view_of(x0);
  py::object inv;
  ArrayView vinv;
  if (!inv_diag_o.is_none()) {
    inv = contiguous(inv_diag_o);
    vinv = view_of(inv);
  }
  if (vb.ndim != 1) msx::require_rank(vb, 1, inv_diag_o.is_none() ? "csr_cg b" : "csr_pcg_jacobi b");
  py::object x = empty_like_out(vb, b, py::make_tuple(vb.shape[0]));
  const ArrayView vx = view_of(x);
  const msx::ExecContext ctx = context_for(vd, 0);
  msx_solver_result res{};
  const ArrayView *pinv = inv_diag_o.is_none() ? nullptr : &vinv;
  if (vd.device >= 0) {
    res = msx::csr_cg(vd, vi, vp, vb, vx0, pinv, vx, n_rows, n_cols, rtol, atol, maxiter,
                      plan_ptr(plan), ctx);
  } else {
    py::gil_scoped_release nogil;
    res = msx::csr_cg(vd, vi, vp, vb, vx0, pinv, vx, n_rows, n_cols, rtol, atol, maxiter, nullptr,
                      ctx);
  }
  return py::make_tuple(x, res.info, res.residual, res.iterations);
}

py::tuple solve_krylov(msx::Krylov kind, py::handle data_o, py::handle indices_o,
                       py::handle indptr_o, py::handle b_o, py::handle x0_o, int64_t n_rows,
                       int64_t n_cols, float rtol, float atol, int64_t maxiter, float shift,
                       py::object plan, int64_t restart = 0,
                       py::object inv_diag_o = py::none()) {
  py::object data = contiguous(data_o), indices = contiguous(indices_o),
             indptr = contiguous(indptr_o), b = contiguous(b_o), x0 = contiguous(x0_o);
  const ArrayView vd = view_of(data), vi = view_of(indices), vp = view_of(indptr), vb = view_of(b),
                  vx0 = view_of(x0);
  py::object inv;
  ArrayView vinv;
  if (!inv_diag_o.is_none()) {
    inv = contiguous(inv_diag_o);
    vinv = view_of(inv);
  }
  const ArrayView *pinv = inv_diag_o.is_none() ? nullptr : &vinv;
  if (vb.ndim != 1)
    msx::require_rank(vb, 1, kind == msx::Krylov::BiCGSTAB ? "csr_bicgstab b"
                             : kind == msx::Krylov::MINRES ? "csr_minres b"
                                                           : "csr_gmres b");
  py::object x = empty_like_out(vb, b, py::make_tuple(vb.shape[0]));
  const ArrayView vx = view_of(x);
  const msx::ExecContext ctx = context_for(vd, 0);
  msx_solver_result res{};
  if (vd.device >= 0) {
    res = msx::csr_krylov(kind, vd, vi, vp, vb, vx0, vx, n_rows, n_cols, rtol, atol, maxiter,
                          shift, plan_ptr(plan), ctx, restart, pinv);
  } else {
    py::gil_scoped_release nogil;
    res = msx::csr_krylov(kind, vd, vi, vp, vb, vx0, vx, n_rows, n_cols, rtol, atol, maxiter,
                          shift, nullptr, ctx, restart, pinv);
  }
  return py::make_tuple(x, res.info, res.residual, res.iterations);
}

py::dict mm_info(const std::string &path) {
  msx_mm_info info{};
  msx::check_status(msx_mm_info_read(path.c_str(), &info), "mmread");
  static const char *formats[] = {"coordinate", "array"};
  static const char *fields[] = {"real", "integer", "complex", "pattern"};
  static const char *syms[] = {"general", "symmetric", "skew-symmetric", "hermitian"};
  py::dict d;
  d["rows"] = info.n_rows;
  d["cols"] = info.n_cols;
  d["entries"] = info.entries;
  d["nnz_bound"] = info.nnz_bound;
  d["format"] = formats[info.format];
  d["field"] = fields[info.field];
  d["symmetry"] = syms[info.symmetry];
  return d;
}

py::object host_empty(int64_t n, py::object dtype) {
  py::dict kw;
  kw["dtype"] = dtype;
  return torch().attr("empty")(py::make_tuple(n), **kw);
}

// (data, indices, indptr, shape) of a Matrix Market file as canonical CSR
// host tensors.
py::tuple mm_read_csr(const std::string &path, py::object dtype, py::object index_dtype,
                      int n_threads) {
  msx_mm_info info{};
  msx::check_status(msx_mm_info_read(path.c_str(), &info), "mmread");
  const std::string vname = dtype_name(dtype), iname = dtype_name(index_dtype);
  const DType vd = dtype_of(vname), id = dtype_of(iname);
  if (!msx::is_value_dtype(vd))
    throw std::invalid_argument("mmread dtype must be float32, float16, bfloat16 or complex64.");
  if (id != DType::Int32 && id != DType::Int64)
    throw std::invalid_argument("mmread index_dtype must be int32 or int64.");
  py::object data = host_empty(std::max<int64_t>(info.nnz_bound, 1), dtype);
  py::object indices = host_empty(std::max<int64_t>(info.nnz_bound, 1), index_dtype);
  py::object indptr = host_empty(info.n_rows + 1, index_dtype);
  const ArrayView vdv = view_of(data), viv = view_of(indices), vpv = view_of(indptr);
  int64_t nnz = 0;
  {
    py::gil_scoped_release nogil;
    msx::check_status(msx_mm_read_csr(path.c_str(), msx::to_vtype(vd), msx::to_itype(id),
                                      info.nnz_bound, vdv.ptr, viv.ptr, vpv.ptr, &nnz, n_threads),
                      "mmread");
  }
  py::object sl = py::module_::import("builtins").attr("slice")(0, nnz);
  return py::make_tuple(data.attr("__getitem__")(sl).attr("clone")(),
                        indices.attr("__getitem__")(sl).attr("clone")(), indptr,
                        py::make_tuple(info.n_rows, info.n_cols));
}

py::object mm_read_dense(const std::string &path, py::object dtype, int n_threads) {
  msx_mm_info info{};
  msx::check_status(msx_mm_info_read(path.c_str(), &info), "mmread");
  const DType vd = dtype_of(dtype_name(dtype));
  if (!msx::is_value_dtype(vd))
    throw std::invalid_argument("mmread dtype must be float32, float16, bfloat16 or complex64.");
  py::object out = host_empty(info.n_rows * info.n_cols, dtype);
  const ArrayView vo = view_of(out);
  {
    py::gil_scoped_release nogil;
    msx::check_status(msx_mm_read_dense(path.c_str(), msx::to_vtype(vd), info.n_rows * info.n_cols,
                                        vo.ptr, n_threads),
                      "mmread");
  }
  return out.attr("reshape")(info.n_rows, info.n_cols);
}

py::dict plan_info(const Plan &plan) {
  msx_plan_info info{};
  msx::check_status(msx_csr_plan_info(plan.p, &info), "csr_plan_info");
  py::dict d;
  d["n_rows"] = info.n_rows;
  d["nnz"] = info.nnz;
  d["block_nnz"] = info.block_nnz;
  d["block_rows"] = info.block_rows;
  d["chunk_nnz"] = info.chunk_nnz;
  d["n_blocks"] = info.n_blocks;
  d["n_bounds"] = info.n_bounds;
  d["n_long_rows"] = info.n_long_rows;
  d["n_chunks"] = info.n_chunks;
  d["device"] = info.device;
  d["plan_bytes"] = info.plan_bytes;
  d["n_slices"] = info.n_slices;
  d["slice_width"] = info.slice_width;
  d["slice_bytes"] = info.slice_bytes;
  d["n_panels"] = info.n_panels;
  d["panel_width"] = info.panel_width;
  d["n_tiles"] = info.n_tiles;
  d["panel_values"] = info.panel_values;
  d["panel_bytes"] = info.panel_bytes;
  d["window_rows"] = info.window_rows;
  return d;
}

py::tuple plan_export(const Plan &plan) {
  msx_plan_info info{};
  msx::check_status(msx_csr_plan_info(plan.p, &info), "csr_plan_export");
  py::dict kw;
  kw["dtype"] = torch().attr("int64");
  py::object blocks = torch().attr("empty")(info.n_bounds + 1, **kw);
  py::object longs = torch().attr("empty")(info.n_long_rows, **kw);
  py::object chunks = torch().attr("empty")(info.n_long_rows + 1, **kw);
  auto ptr = [](py::object &t) {
    return reinterpret_cast<int64_t *>(t.attr("data_ptr")().cast<uintptr_t>());
  };
  msx::check_status(msx_csr_plan_export(plan.p, ptr(blocks), info.n_long_rows ? ptr(longs) : nullptr,
                                        ptr(chunks)),
                    "csr_plan_export");
  return py::make_tuple(blocks, longs, chunks);
}

py::dict compiled_capabilities() {
  py::dict info;
  info["extension"] = true;
  info["cpu"] = true;
  info["metal"] = false;
  info["accelerate"] = false;
  info["accelerate_framework"] = false;
  info["cuda"] = false;
  info["rocm"] = true;
  info["platform"] = "linux";
  info["architecture"] = "gfx950";
  info["abi_version"] = msx_abi_version();
  return info;
}

}  // namespace

PYBIND11_MODULE(_ext, m) {
  m.doc() = "MI355X (gfx950) CSR sparse x dense primitives for mlx_sparse";

  py::class_<Plan, std::shared_ptr<Plan>>(m, "CSRPlan")
      .def_readonly("n_rows", &Plan::n_rows)
      .def_readonly("nnz", &Plan::nnz)
      .def_readonly("index_dtype", &Plan::index_dtype)
      .def_readonly("device", &Plan::device)
      .def("info", &plan_info, "Plan summary (block and long-row counts, sizes).")
      .def("refresh", &plan_refresh, py::arg("data"),
           "The values changed (indices and indptr did not): rewrite the plan's copies "
           "from data, which the plan is bound to from now on.")
      .def("export", &plan_export,
           "Host copies (int64 tensors) of bounds, long_rows and long_chunk_begin.");

  m.def("_compiled_capabilities", &compiled_capabilities,
        "Return compile-time native backend facts for capability reporting.");
  m.def("csr_plan", &make_plan, py::arg("indptr"), py::arg("n_rows"), py::arg("nnz"),
        py::arg("block_nnz") = 0, py::arg("data") = py::none(), py::arg("indices") = py::none(),
        py::arg("n_cols") = -1, py::arg("slice_mode") = 0,
        "Build a row-block plan from a GPU indptr; with data/indices, a plan bound to the "
        "matrix (slice_mode 0 auto, 1 off, 2 column slices per XCD, 3 LDS column panels).");
  m.def("csr_matvec", &csr_matvec, py::arg("data"), py::arg("indices"), py::arg("indptr"),
        py::arg("x"), py::arg("n_rows"), py::arg("n_cols"), py::arg("plan") = py::none(),
        py::arg("n_threads") = 0, "Multiply CSR buffers by a dense vector.");
  m.def("csr_matmul", &csr_matmul, py::arg("data"), py::arg("indices"), py::arg("indptr"),
        py::arg("rhs"), py::arg("n_rows"), py::arg("n_cols"), py::arg("plan") = py::none(),
        py::arg("n_threads") = 0, "Multiply CSR buffers by a dense matrix.");
  m.def("csr_batched_matvec", &csr_batched_matvec, py::arg("data"), py::arg("indices"),
        py::arg("indptr"), py::arg("rhs"), py::arg("n_rows"), py::arg("n_cols"),
        py::arg("n_threads") = 0, "Multiply CSR buffers by a batch of dense vectors (batch, n_cols).");
  m.def("csr_batched_matmul", &csr_batched_matmul, py::arg("data"), py::arg("indices"),
        py::arg("indptr"), py::arg("rhs"), py::arg("n_rows"), py::arg("n_cols"),
        py::arg("n_threads") = 0,
        "Multiply CSR buffers by a batch of dense matrices (batch, n_cols, k).");
  m.def("csr_transpose", &csr_transpose, py::arg("data"), py::arg("indices"), py::arg("indptr"),
        py::arg("n_rows"), py::arg("n_cols"),
        "CSR buffers of the transpose: (data, indices, indptr), shape (n_cols, n_rows).");
  m.def("csr_transpose_positions", &csr_transpose_positions, py::arg("indices"),
        py::arg("indptr"), py::arg("n_rows"), py::arg("n_cols"),
        "(t_pos, t_indices, t_indptr): the transpose's structure and the position of A each "
        "entry holds (int32, -1 past t_indptr[n_cols]).");
  m.def("csr_transpose_values", &csr_transpose_values, py::arg("data"), py::arg("positions"),
        py::arg("conjugate"), py::arg("out"),
        "out[i] = data[positions[i]] (conjugated on request), in place.");
  m.def("csr_transpose_layout", &csr_transpose_layout, py::arg("positions"), py::arg("like"),
        "(slot1, src1, slot2): layout of the two-pass regather of values of like's dtype.");
  m.def("csr_transpose_values_layout", &csr_transpose_values_layout, py::arg("data"),
        py::arg("slot1"), py::arg("src1"), py::arg("slot2"), py::arg("conjugate"),
        py::arg("scratch"), py::arg("out"),
        "out = data regathered through a csr_transpose_layout layout, in place.");
  m.def("csr_matvec_transpose", &csr_matvec_transpose, py::arg("data"), py::arg("indices"),
        py::arg("indptr"), py::arg("x"), py::arg("n_rows"), py::arg("n_cols"),
        py::arg("n_threads") = 0, "A^T x for CSR buffers of shape (n_rows, n_cols).");
  m.def("csr_matmul_transpose", &csr_matmul_transpose, py::arg("data"), py::arg("indices"),
        py::arg("indptr"), py::arg("rhs"), py::arg("n_rows"), py::arg("n_cols"),
        py::arg("n_threads") = 0, "A^T X for CSR buffers of shape (n_rows, n_cols).");
  m.def("csr_matvec_data_vjp", &csr_matvec_data_vjp, py::arg("indices"), py::arg("indptr"),
        py::arg("x"), py::arg("cotangent"), py::arg("n_rows"), py::arg("n_cols"),
        py::arg("n_threads") = 0, py::arg("plan") = py::none(),
        "Gradient of A x with respect to the stored values (a GPU plan of the matrix may "
        "serve the gather of x).");
  m.def("csr_matmul_data_vjp", &csr_matmul_data_vjp, py::arg("indices"), py::arg("indptr"),
        py::arg("rhs"), py::arg("cotangent"), py::arg("n_rows"), py::arg("n_cols"),
        py::arg("n_threads") = 0, "Gradient of A X with respect to the stored values.");
  m.def(
      "csr_cg",
      [](py::handle data, py::handle indices, py::handle indptr, py::handle b, py::handle x0,
         int64_t n_rows, int64_t n_cols, float rtol, float atol, int64_t maxiter, py::object plan) {
        return solve_cg(data, indices, indptr, b, x0, py::none(), n_rows, n_cols, rtol, atol,
                        maxiter, plan);
      },
      py::arg("data"), py::arg("indices"), py::arg("indptr"), py::arg("b"), py::arg("x0"),
      py::arg("n_rows"), py::arg("n_cols"), py::arg("rtol"), py::arg("atol"), py::arg("maxiter"),
      py::arg("plan") = py::none(),
      "Conjugate gradients: (x, info, residual, iterations).");
  m.def(
      "csr_pcg_jacobi",
      [](py::handle data, py::handle indices, py::handle indptr, py::handle b, py::handle x0,
         py::handle inv_diag, int64_t n_rows, int64_t n_cols, float rtol, float atol,
         int64_t maxiter, py::object plan) {
        return solve_cg(data, indices, indptr, b, x0, py::reinterpret_borrow<py::object>(inv_diag),
                        n_rows, n_cols, rtol, atol, maxiter, plan);
      },
      py::arg("data"), py::arg("indices"), py::arg("indptr"), py::arg("b"), py::arg("x0"),
      py::arg("inv_diag"), py::arg("n_rows"), py::arg("n_cols"), py::arg("rtol"),
      py::arg("atol"), py::arg("maxiter"), py::arg("plan") = py::none(),
      "Jacobi-preconditioned conjugate gradients: (x, info, residual, iterations).");
  m.def(
      "csr_bicgstab",
      [](py::handle data, py::handle indices, py::handle indptr, py::handle b, py::handle x0,
         int64_t n_rows, int64_t n_cols, float rtol, float atol, int64_t maxiter, py::object plan) {
        return solve_krylov(msx::Krylov::BiCGSTAB, data, indices, indptr, b, x0, n_rows, n_cols,
                            rtol, atol, maxiter, 0.0f, plan);
      },
      py::arg("data"), py::arg("indices"), py::arg("indptr"), py::arg("b"), py::arg("x0"),
      py::arg("n_rows"), py::arg("n_cols"), py::arg("rtol"), py::arg("atol"), py::arg("maxiter"),
      py::arg("plan") = py::none(), "BiCGSTAB: (x, info, residual, iterations).");
  m.def(
      "csr_bicgstab_jacobi",
      [](py::handle data, py::handle indices, py::handle indptr, py::handle b, py::handle x0,
         py::handle inv_diag, int64_t n_rows, int64_t n_cols, float rtol, float atol,
         int64_t maxiter, py::object plan) {
        return solve_krylov(msx::Krylov::BiCGSTAB, data, indices, indptr, b, x0, n_rows, n_cols,
                            rtol, atol, maxiter, 0.0f, plan, 0,
                            py::reinterpret_borrow<py::object>(inv_diag));
      },
      py::arg("data"), py::arg("indices"), py::arg("indptr"), py::arg("b"), py::arg("x0"),
      py::arg("inv_diag"), py::arg("n_rows"), py::arg("n_cols"), py::arg("rtol"),
      py::arg("atol"), py::arg("maxiter"), py::arg("plan") = py::none(),
      "Jacobi-preconditioned BiCGSTAB: (x, info, residual, iterations).");
  m.def(
      "csr_minres",
      [](py::handle data, py::handle indices, py::handle indptr, py::handle b, py::handle x0,
         int64_t n_rows, int64_t n_cols, float rtol, float atol, int64_t maxiter, float shift,
         py::object plan) {
        return solve_krylov(msx::Krylov::MINRES, data, indices, indptr, b, x0, n_rows, n_cols,
                            rtol, atol, maxiter, shift, plan);
      },
      py::arg("data"), py::arg("indices"), py::arg("indptr"), py::arg("b"), py::arg("x0"),
      py::arg("n_rows"), py::arg("n_cols"), py::arg("rtol"), py::arg("atol"), py::arg("maxiter"),
      py::arg("shift") = 0.0f, py::arg("plan") = py::none(),
      "MINRES on (A - shift I) x = b: (x, info, residual, iterations).");
  m.def(
      "csr_minres_jacobi",
      [](py::handle data, py::handle indices, py::handle indptr, py::handle b, py::handle x0,
         py::handle inv_diag, int64_t n_rows, int64_t n_cols, float rtol, float atol,
         int64_t maxiter, float shift, py::object plan) {
        return solve_krylov(msx::Krylov::MINRES, data, indices, indptr, b, x0, n_rows, n_cols,
                            rtol, atol, maxiter, shift, plan, 0,
                            py::reinterpret_borrow<py::object>(inv_diag));
      },
      py::arg("data"), py::arg("indices"), py::arg("indptr"), py::arg("b"), py::arg("x0"),
      py::arg("inv_diag"), py::arg("n_rows"), py::arg("n_cols"), py::arg("rtol"),
      py::arg("atol"), py::arg("maxiter"), py::arg("shift") = 0.0f, py::arg("plan") = py::none(),
      "Jacobi-preconditioned MINRES on (A - shift I) x = b: (x, info, residual, iterations).");
  m.def(
      "csr_gmres",
      [](py::handle data, py::handle indices, py::handle indptr, py::handle b, py::handle x0,
         int64_t n_rows, int64_t n_cols, float rtol, float atol, int64_t restart, int64_t maxiter,
         py::object plan) {
        return solve_krylov(msx::Krylov::GMRES, data, indices, indptr, b, x0, n_rows, n_cols,
                            rtol, atol, maxiter, 0.0f, plan, restart);
      },
      py::arg("data"), py::arg("indices"), py::arg("indptr"), py::arg("b"), py::arg("x0"),
      py::arg("n_rows"), py::arg("n_cols"), py::arg("rtol"), py::arg("atol"), py::arg("restart"),
      py::arg("maxiter"), py::arg("plan") = py::none(),
      "Restarted GMRES: (x, info, residual, iterations).");
  m.def(
      "csr_gmres_jacobi",
      [](py::handle data, py::handle indices, py::handle indptr, py::handle b, py::handle x0,
         py::handle inv_diag, int64_t n_rows, int64_t n_cols, float rtol, float atol,
         int64_t restart, int64_t maxiter, py::object plan) {
        return solve_krylov(msx::Krylov::GMRES, data, indices, indptr, b, x0, n_rows, n_cols,
                            rtol, atol, maxiter, 0.0f, plan, restart,
                            py::reinterpret_borrow<py::object>(inv_diag));
      },
      py::arg("data"), py::arg("indices"), py::arg("indptr"), py::arg("b"), py::arg("x0"),
      py::arg("inv_diag"), py::arg("n_rows"), py::arg("n_cols"), py::arg("rtol"),
      py::arg("atol"), py::arg("restart"), py::arg("maxiter"), py::arg("plan") = py::none(),
      "Jacobi-preconditioned restarted GMRES: (x, info, residual, iterations).");
  m.def("mm_info", &mm_info, py::arg("path"), "Header of a Matrix Market file.");
  m.def("mm_read_csr", &mm_read_csr, py::arg("path"), py::arg("dtype"), py::arg("index_dtype"),
        py::arg("n_threads") = 0,
        "Matrix Market file -> (data, indices, indptr, shape), canonical CSR host tensors.");
  m.def("mm_read_dense", &mm_read_dense, py::arg("path"), py::arg("dtype"),
        py::arg("n_threads") = 0, "Matrix Market file -> dense row-major host tensor.");
  m.def("cpu_worker_count", &msx_cpu_worker_count, "Resolved CPU worker count.");
  m.def(
      "cpu_ranges",
      [](std::vector<int64_t> work, int parts) {
        std::vector<int64_t> out(2 * static_cast<size_t>(std::max(parts, 1)));
        int64_t n = 0;
        msx::check_status(msx_cpu_ranges(work.data(), static_cast<int64_t>(work.size()), parts,
                                         out.data(), &n),
                          "cpu_ranges");
        std::vector<std::pair<int64_t, int64_t>> r;
        for (int64_t i = 0; i < n; ++i) r.emplace_back(out[2 * i], out[2 * i + 1]);
        return r;
      },
      py::arg("work"), py::arg("parts"), "Row ranges the CPU path splits work into.");
  m.def("device_count", []() {
    int c = 0;
    msx::check_status(msx_device_count(&c), "device_count");
    return c;
  });
  m.def("abi_version", &msx_abi_version);
}
