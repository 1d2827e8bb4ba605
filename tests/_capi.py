"""ctypes front end of libmsx_sparse (include/msx_sparse.h) for the tests:
the GPU parity tests call the HIP path through exactly this C ABI."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "msx_sparse.h"
LIB = ROOT / "mlx-sparse_amd" / "mlx_sparse" / "libmsx_sparse.so"

VT = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2, torch.complex64: 3}
IT = {torch.int32: 0, torch.int64: 1}
OK, EINVAL, ETYPE, EHIP, ENOMEM = range(5)


class PlanInfo(ctypes.Structure):
    _fields_ = [(name, ctypes.c_int64) for name in (
        "n_rows", "nnz", "block_nnz", "block_rows", "chunk_nnz", "n_blocks", "n_bounds", "n_long_rows",
        "n_chunks", "device", "plan_bytes", "n_slices", "slice_width", "slice_bytes",
        "n_panels", "panel_width", "n_tiles", "panel_values", "panel_bytes", "window_rows")]


class PlanOptions(ctypes.Structure):
    _fields_ = [("block_nnz", ctypes.c_int64), ("slice_mode", ctypes.c_int32),
                ("reserved", ctypes.c_int32)]


SLICE_AUTO, SLICE_OFF, SLICE_ON, SLICE_PANELS = 0, 1, 2, 3


class SolverResult(ctypes.Structure):
    _fields_ = [("info", ctypes.c_int32), ("iterations", ctypes.c_int32),
                ("residual", ctypes.c_float), ("reserved", ctypes.c_int32)]


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(msx_\w+)\s*\(", text, re.M)))


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        L = ctypes.CDLL(str(LIB))
        i64, vp, ci = ctypes.c_int64, ctypes.c_void_p, ctypes.c_int
        L.msx_abi_version.restype = ci
        L.msx_last_error.restype = ctypes.c_char_p
        L.msx_device_count.argtypes = [ctypes.POINTER(ci)]
        L.msx_csr_plan_create.argtypes = [ci, i64, i64, vp, i64, vp, ctypes.POINTER(vp)]
        L.msx_csr_plan_create_bound.argtypes = [ci, ci, i64, i64, i64, vp, vp, vp,
                                                ctypes.POINTER(PlanOptions), vp, ctypes.POINTER(vp)]
        L.msx_csr_plan_destroy.argtypes = [vp]
        L.msx_csr_plan_refresh.argtypes = [vp, vp, vp]
        L.msx_csr_transpose_positions.argtypes = [ci, i64, i64, i64, vp, vp, vp, vp, vp, vp]
        L.msx_csr_transpose_values.argtypes = [ci, i64, vp, vp, ci, vp, vp]
        L.msx_csr_transpose_layout.argtypes = [ci, i64, vp, vp, vp, vp, vp]
        L.msx_csr_transpose_values_layout.argtypes = [ci, i64, vp, vp, vp, vp, ci, vp, vp, vp]
        L.msx_csr_plan_info.argtypes = [vp, ctypes.POINTER(PlanInfo)]
        L.msx_csr_plan_export.argtypes = [vp, vp, vp, vp]
        L.msx_csr_plan_export_panels.argtypes = [vp, vp, vp, vp]
        L.msx_csr_spmv.argtypes = [ci, ci, i64, i64, i64, vp, vp, vp, vp, vp, vp, vp]
        L.msx_csr_spmm.argtypes = [ci, ci, i64, i64, i64, vp, vp, vp, i64, vp, i64, vp, i64, vp, vp]
        L.msx_csr_batched_spmv.argtypes = [ci, ci, i64, i64, i64, vp, vp, vp, i64, vp, i64, vp,
                                           i64, vp]
        L.msx_csr_batched_spmm.argtypes = [ci, ci, i64, i64, i64, vp, vp, vp, i64, i64, vp, i64,
                                           i64, vp, i64, i64, vp]
        L.msx_csr_batched_spmv_cpu.argtypes = [ci, ci, i64, i64, i64, vp, vp, vp, i64, vp, vp, ci]
        L.msx_csr_batched_spmm_cpu.argtypes = [ci, ci, i64, i64, i64, vp, vp, vp, i64, i64, vp,
                                               vp, ci]
        L.msx_csr_spmv_cpu.argtypes = [ci, ci, i64, i64, i64, vp, vp, vp, vp, vp, ci]
        L.msx_csr_spmm_cpu.argtypes = [ci, ci, i64, i64, i64, vp, vp, vp, i64, vp, vp, ci]
        L.msx_csr_transpose.argtypes = [ci, ci, i64, i64, i64, vp, vp, vp, vp, vp, vp, vp]
        L.msx_csr_transpose_cpu.argtypes = [ci, ci, i64, i64, i64, vp, vp, vp, vp, vp, vp]
        L.msx_csr_spmv_transpose.argtypes = [ci, ci, i64, i64, i64, vp, vp, vp, vp, vp, vp]
        L.msx_csr_spmv_transpose_noalloc.argtypes = [ci, ci, i64, i64, i64, vp, vp, vp, vp, vp,
                                                     vp]
        L.msx_csr_spmm_transpose.argtypes = [ci, ci, i64, i64, i64, vp, vp, vp, i64, vp, i64, vp,
                                             i64, vp]
        L.msx_csr_spmv_transpose_cpu.argtypes = [ci, ci, i64, i64, i64, vp, vp, vp, vp, vp, ci]
        L.msx_csr_spmm_transpose_cpu.argtypes = [ci, ci, i64, i64, i64, vp, vp, vp, i64, vp, vp,
                                                 ci]
        L.msx_csr_spmv_data_vjp.argtypes = [ci, ci, i64, i64, i64, vp, vp, vp, vp, vp, vp, vp]
        L.msx_csr_spmm_data_vjp.argtypes = [ci, ci, i64, i64, i64, vp, vp, i64, vp, i64, vp, i64,
                                            vp, vp]
        L.msx_csr_spmv_data_vjp_cpu.argtypes = [ci, ci, i64, i64, i64, vp, vp, vp, vp, vp, ci]
        L.msx_csr_spmm_data_vjp_cpu.argtypes = [ci, ci, i64, i64, i64, vp, vp, i64, vp, vp, vp,
                                                ci]
        f32 = ctypes.c_float
        L.msx_csr_cg.argtypes = [ci, i64, i64, vp, vp, vp, vp, vp, vp, f32, f32, i64, vp, vp, vp]
        L.msx_csr_pcg_jacobi.argtypes = [ci, i64, i64, vp, vp, vp, vp, vp, vp, vp, f32, f32, i64,
                                         vp, vp, vp]
        L.msx_csr_cg_cpu.argtypes = [ci, i64, i64, vp, vp, vp, vp, vp, vp, f32, f32, i64, vp]
        L.msx_csr_pcg_jacobi_cpu.argtypes = [ci, i64, i64, vp, vp, vp, vp, vp, vp, vp, f32, f32,
                                             i64, vp]
        L.msx_csr_bicgstab.argtypes = [ci, i64, i64, vp, vp, vp, vp, vp, vp, f32, f32, i64, vp,
                                       vp, vp]
        L.msx_csr_minres.argtypes = [ci, i64, i64, vp, vp, vp, vp, vp, vp, f32, f32, i64, f32, vp,
                                     vp, vp]
        L.msx_csr_bicgstab_cpu.argtypes = [ci, i64, i64, vp, vp, vp, vp, vp, vp, f32, f32, i64, vp]
        L.msx_csr_bicgstab_jacobi.argtypes = [ci, i64, i64, vp, vp, vp, vp, vp, vp, vp, f32, f32,
                                              i64, vp, vp, vp]
        L.msx_csr_bicgstab_jacobi_cpu.argtypes = [ci, i64, i64, vp, vp, vp, vp, vp, vp, vp, f32,
                                                  f32, i64, vp]
        L.msx_csr_minres_cpu.argtypes = [ci, i64, i64, vp, vp, vp, vp, vp, vp, f32, f32, i64, f32,
                                         vp]
        L.msx_csr_minres_jacobi.argtypes = [ci, i64, i64, vp, vp, vp, vp, vp, vp, vp, f32, f32,
                                            i64, f32, vp, vp, vp]
        L.msx_csr_minres_jacobi_cpu.argtypes = [ci, i64, i64, vp, vp, vp, vp, vp, vp, vp, f32, f32,
                                                i64, f32, vp]
        L.msx_csr_gmres.argtypes = [ci, i64, i64, vp, vp, vp, vp, vp, vp, f32, f32, i64, i64, vp,
                                    vp, vp]
        L.msx_csr_gmres_cpu.argtypes = [ci, i64, i64, vp, vp, vp, vp, vp, vp, f32, f32, i64, i64,
                                        vp]
        L.msx_csr_gmres_jacobi.argtypes = [ci, i64, i64, vp, vp, vp, vp, vp, vp, vp, f32, f32, i64,
                                           i64, vp, vp, vp]
        L.msx_csr_gmres_jacobi_cpu.argtypes = [ci, i64, i64, vp, vp, vp, vp, vp, vp, vp, f32, f32,
                                               i64, i64, vp]
        L.msx_cpu_worker_count.restype = ci
        L.msx_cpu_ranges.argtypes = [vp, i64, ci, vp, ctypes.POINTER(i64)]
        for name in ("msx_device_count", "msx_csr_plan_create", "msx_csr_plan_create_bound",
                     "msx_csr_plan_destroy", "msx_csr_plan_refresh",
                     "msx_csr_transpose_positions", "msx_csr_transpose_values",
                     "msx_csr_transpose_layout", "msx_csr_transpose_values_layout",
                     "msx_csr_plan_info", "msx_csr_plan_export", "msx_csr_plan_export_panels",
                     "msx_csr_spmv", "msx_csr_spmm", "msx_csr_batched_spmv",
                     "msx_csr_batched_spmm", "msx_csr_batched_spmv_cpu",
                     "msx_csr_batched_spmm_cpu",
                     "msx_csr_spmv_cpu", "msx_csr_spmm_cpu", "msx_cpu_ranges",
                     "msx_csr_transpose", "msx_csr_transpose_cpu", "msx_csr_spmv_transpose",
                     "msx_csr_spmv_transpose_noalloc",
                     "msx_csr_spmm_transpose", "msx_csr_spmv_transpose_cpu",
                     "msx_csr_spmm_transpose_cpu", "msx_csr_spmv_data_vjp",
                     "msx_csr_spmm_data_vjp", "msx_csr_spmv_data_vjp_cpu",
                     "msx_csr_spmm_data_vjp_cpu", "msx_csr_cg", "msx_csr_pcg_jacobi",
                     "msx_csr_cg_cpu", "msx_csr_pcg_jacobi_cpu", "msx_csr_bicgstab",
                     "msx_csr_minres", "msx_csr_bicgstab_cpu", "msx_csr_minres_cpu",
                     "msx_csr_bicgstab_jacobi", "msx_csr_bicgstab_jacobi_cpu",
                     "msx_csr_minres_jacobi", "msx_csr_minres_jacobi_cpu",
                     "msx_csr_gmres", "msx_csr_gmres_cpu", "msx_csr_gmres_jacobi",
                     "msx_csr_gmres_jacobi_cpu"):
            getattr(L, name).restype = ci
        _lib = L
    return _lib


def last_error() -> str:
    return lib().msx_last_error().decode()


def _p(t):
    return None if t is None else t.data_ptr()


def _stream():
    return torch.cuda.current_stream().cuda_stream


class Plan:
    def __init__(self, indptr: torch.Tensor, n_rows: int, nnz: int, block_nnz: int = 0, *,
                 data=None, indices=None, n_cols: int = 0, slice_mode: int | None = None):
        self.ptr = ctypes.c_void_p()
        if data is None:
            st = lib().msx_csr_plan_create(IT[indptr.dtype], n_rows, nnz, _p(indptr), block_nnz,
                                           _stream(), ctypes.byref(self.ptr))
        else:
            opts = PlanOptions(block_nnz, SLICE_AUTO if slice_mode is None else slice_mode, 0)
            self._keep = (data, indices, indptr)
            st = lib().msx_csr_plan_create_bound(VT[data.dtype], IT[indptr.dtype], n_rows, n_cols,
                                                 nnz, _p(data), _p(indices), _p(indptr),
                                                 ctypes.byref(opts), _stream(), ctypes.byref(self.ptr))
        if st != OK:
            raise RuntimeError(f"plan_create: {st} {last_error()}")

    def info(self) -> PlanInfo:
        info = PlanInfo()
        assert lib().msx_csr_plan_info(self.ptr, ctypes.byref(info)) == OK
        return info

    def export(self):
        info = self.info()
        blocks = torch.empty(info.n_bounds + 1, dtype=torch.int64)
        longs = torch.empty(max(info.n_long_rows, 1), dtype=torch.int64)
        chunks = torch.empty(info.n_long_rows + 1, dtype=torch.int64)
        st = lib().msx_csr_plan_export(self.ptr, _p(blocks), _p(longs), _p(chunks))
        assert st == OK, last_error()
        return blocks.numpy(), longs[: info.n_long_rows].numpy(), chunks.numpy()

    def refresh(self, data):
        """The values changed: rewrite the plan's copies from ``data``."""
        st = lib().msx_csr_plan_refresh(self.ptr, _p(data), _stream())
        if st != OK:
            raise RuntimeError(f"plan_refresh: {st} {last_error()}")
        if getattr(self, "_keep", None) is not None:
            self._keep = (data,) + self._keep[1:]

    def export_panels(self):
        info = self.info()
        tb = torch.empty(max(info.n_tiles, 1), dtype=torch.int64)
        te = torch.empty(max(info.n_tiles, 1), dtype=torch.int64)
        seg = torch.empty(info.n_panels * info.n_tiles + 1, dtype=torch.int64)
        st = lib().msx_csr_plan_export_panels(self.ptr, _p(tb), _p(te), _p(seg))
        assert st == OK, last_error()
        return tb[: info.n_tiles].numpy(), te[: info.n_tiles].numpy(), seg.numpy()

    def close(self):
        if self.ptr:
            lib().msx_csr_plan_destroy(self.ptr)
            self.ptr = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def spmv(data, indices, indptr, x, n_rows, n_cols, plan: Plan | None = None, y=None):
    if y is None:
        y = torch.empty(n_rows, dtype=data.dtype, device=data.device)
    st = lib().msx_csr_spmv(VT[data.dtype], IT[indices.dtype], n_rows, n_cols, data.numel(),
                            _p(data), _p(indices), _p(indptr), _p(x), _p(y),
                            plan.ptr if plan else None, _stream())
    if st != OK:
        raise RuntimeError(f"msx_csr_spmv: {st} {last_error()}")
    return y


def spmm(data, indices, indptr, X, n_rows, n_cols, Y=None, ldx=None, ldy=None,
         plan: Plan | None = None):
    k = X.shape[1]
    if Y is None:
        Y = torch.empty((n_rows, k), dtype=data.dtype, device=data.device)
    st = lib().msx_csr_spmm(VT[data.dtype], IT[indices.dtype], n_rows, n_cols, data.numel(),
                            _p(data), _p(indices), _p(indptr), k, _p(X),
                            ldx if ldx is not None else X.stride(0), _p(Y),
                            ldy if ldy is not None else Y.stride(0),
                            plan.ptr if plan is not None else None, _stream())
    if st != OK:
        raise RuntimeError(f"msx_csr_spmm: {st} {last_error()}")
    return Y


def batched_spmv(data, indices, indptr, X, n_rows, n_cols, Y=None, ldx=None, ldy=None):
    """X: (batch, >= n_cols) rows of stride ldx; Y: (batch, >= n_rows)."""
    batch = X.shape[0]
    if Y is None:
        Y = torch.empty((batch, n_rows), dtype=data.dtype, device=data.device)
    st = lib().msx_csr_batched_spmv(VT[data.dtype], IT[indices.dtype], n_rows, n_cols,
                                    data.numel(), _p(data), _p(indices), _p(indptr), batch,
                                    _p(X), ldx if ldx is not None else X.stride(0), _p(Y),
                                    ldy if ldy is not None else Y.stride(0), _stream())
    if st != OK:
        raise RuntimeError(f"msx_csr_batched_spmv: {st} {last_error()}")
    return Y


def batched_spmm(data, indices, indptr, X, n_rows, n_cols, Y=None):
    """X: (batch, n_cols, k) with any batch/row strides of a torch view."""
    batch, _, k = X.shape
    if Y is None:
        Y = torch.empty((batch, n_rows, k), dtype=data.dtype, device=data.device)
    st = lib().msx_csr_batched_spmm(VT[data.dtype], IT[indices.dtype], n_rows, n_cols,
                                    data.numel(), _p(data), _p(indices), _p(indptr), batch, k,
                                    _p(X), X.stride(0), X.stride(1), _p(Y), Y.stride(0),
                                    Y.stride(1), _stream())
    if st != OK:
        raise RuntimeError(f"msx_csr_batched_spmm: {st} {last_error()}")
    return Y


def _check(st, name):
    if st != OK:
        raise RuntimeError(f"{name}: {st} {last_error()}")


def _is_cpu(t):
    return t.device.type == "cpu"


def transpose(data, indices, indptr, n_rows, n_cols):
    """CSR of A^T: (t_data, t_indices, t_indptr) on data's device."""
    nnz = data.numel()
    td = torch.empty(nnz, dtype=data.dtype, device=data.device)
    ti = torch.empty(nnz, dtype=indices.dtype, device=data.device)
    tp = torch.empty(n_cols + 1, dtype=indptr.dtype, device=data.device)
    args = (VT[data.dtype], IT[indices.dtype], n_rows, n_cols, nnz, _p(data), _p(indices),
            _p(indptr), _p(td), _p(ti), _p(tp))
    if _is_cpu(data):
        _check(lib().msx_csr_transpose_cpu(*args), "msx_csr_transpose_cpu")
    else:
        _check(lib().msx_csr_transpose(*args, _stream()), "msx_csr_transpose")
    return td, ti, tp


def transpose_positions(indices, indptr, n_rows, n_cols):
    """(t_pos int32, t_indices, t_indptr) of A^T on the GPU."""
    nnz = indices.numel()
    pos = torch.empty(nnz, dtype=torch.int32, device=indices.device)
    ti = torch.empty(nnz, dtype=indices.dtype, device=indices.device)
    tp = torch.empty(n_cols + 1, dtype=indptr.dtype, device=indices.device)
    _check(lib().msx_csr_transpose_positions(IT[indices.dtype], n_rows, n_cols, nnz, _p(indices),
                                             _p(indptr), _p(pos), _p(ti), _p(tp), _stream()),
           "msx_csr_transpose_positions")
    return pos, ti, tp


def transpose_values(data, pos, out, conjugate=False):
    _check(lib().msx_csr_transpose_values(VT[data.dtype], data.numel(), _p(data), _p(pos),
                                          1 if conjugate else 0, _p(out), _stream()),
           "msx_csr_transpose_values")
    return out


def transpose_layout(pos, vtype):
    """(slot1, src1, slot2) of the two-pass regather of values of dtype `vtype`."""
    nnz = pos.numel()
    slot1 = torch.empty(nnz, dtype=torch.int16, device=pos.device)
    src1 = torch.empty(nnz, dtype=torch.int32, device=pos.device)
    slot2 = torch.empty(nnz, dtype=torch.int16, device=pos.device)
    _check(lib().msx_csr_transpose_layout(VT[vtype], nnz, _p(pos), _p(slot1), _p(src1), _p(slot2),
                                          _stream()), "msx_csr_transpose_layout")
    return slot1, src1, slot2


def transpose_values_layout(data, layout, out, conjugate=False, scratch=None):
    slot1, src1, slot2 = layout
    scratch = torch.empty_like(data) if scratch is None else scratch
    _check(lib().msx_csr_transpose_values_layout(VT[data.dtype], data.numel(), _p(data), _p(slot1),
                                                 _p(src1), _p(slot2), 1 if conjugate else 0,
                                                 _p(scratch), _p(out), _stream()),
           "msx_csr_transpose_values_layout")
    return out


def spmv_transpose(data, indices, indptr, x, n_rows, n_cols, n_threads=1):
    y = torch.empty(n_cols, dtype=data.dtype, device=data.device)
    head = (VT[data.dtype], IT[indices.dtype], n_rows, n_cols, data.numel(), _p(data),
            _p(indices), _p(indptr), _p(x), _p(y))
    if _is_cpu(data):
        _check(lib().msx_csr_spmv_transpose_cpu(*head, n_threads), "msx_csr_spmv_transpose_cpu")
    else:
        _check(lib().msx_csr_spmv_transpose(*head, _stream()), "msx_csr_spmv_transpose")
    return y


def spmm_transpose(data, indices, indptr, X, n_rows, n_cols, n_threads=1, Y=None, ldy=None):
    k = X.shape[1]
    if Y is None:
        Y = torch.empty((n_cols, k), dtype=data.dtype, device=data.device)
    head = (VT[data.dtype], IT[indices.dtype], n_rows, n_cols, data.numel(), _p(data),
            _p(indices), _p(indptr), k, _p(X))
    if _is_cpu(data):
        _check(lib().msx_csr_spmm_transpose_cpu(*head, _p(Y), n_threads),
               "msx_csr_spmm_transpose_cpu")
    else:
        _check(lib().msx_csr_spmm_transpose(*head, X.stride(0), _p(Y),
                                            ldy if ldy is not None else Y.stride(0), _stream()),
               "msx_csr_spmm_transpose")
    return Y


def spmv_data_vjp(indices, indptr, x, cot, n_rows, n_cols, n_threads=1, plan=None):
    nnz = indices.numel()
    out = torch.empty(nnz, dtype=x.dtype, device=x.device)
    head = (VT[x.dtype], IT[indices.dtype], n_rows, n_cols, nnz, _p(indices), _p(indptr),
            _p(x), _p(cot), _p(out))
    if _is_cpu(x):
        _check(lib().msx_csr_spmv_data_vjp_cpu(*head, n_threads), "msx_csr_spmv_data_vjp_cpu")
    else:
        _check(lib().msx_csr_spmv_data_vjp(*head, plan.ptr if plan is not None else None,
                                           _stream()), "msx_csr_spmv_data_vjp")
    return out


def spmm_data_vjp(indices, indptr, X, cot, n_rows, n_cols, n_threads=1):
    nnz = indices.numel()
    k = X.shape[1]
    out = torch.empty(nnz, dtype=X.dtype, device=X.device)
    it = IT[indices.dtype]
    if _is_cpu(X):
        _check(lib().msx_csr_spmm_data_vjp_cpu(VT[X.dtype], it, n_rows, n_cols, nnz,
                                               _p(indices), _p(indptr), k, _p(X), _p(cot),
                                               _p(out), n_threads),
               "msx_csr_spmm_data_vjp_cpu")
    else:
        _check(lib().msx_csr_spmm_data_vjp(VT[X.dtype], it, n_rows, n_cols, nnz, _p(indices),
                                           _p(indptr), k, _p(X), X.stride(0), _p(cot),
                                           cot.stride(0), _p(out), _stream()),
               "msx_csr_spmm_data_vjp")
    return out


def cg(data, indices, indptr, b, x0=None, *, rtol=1e-5, atol=0.0, maxiter=None, plan=None,
       inv_diag=None):
    """(x, info, residual, iterations) through msx_csr_cg[_cpu] or the
    Jacobi-preconditioned variant when inv_diag is given."""
    n = b.numel()
    x0 = torch.zeros_like(b) if x0 is None else x0
    x = torch.empty_like(b)
    maxiter = 10 * n if maxiter is None else maxiter
    res = SolverResult()
    it = IT[indices.dtype]
    L = lib()
    if b.device.type == "cpu":
        if inv_diag is None:
            st = L.msx_csr_cg_cpu(it, n, data.numel(), _p(data), _p(indices), _p(indptr), _p(b),
                                  _p(x0), _p(x), rtol, atol, maxiter, ctypes.byref(res))
        else:
            st = L.msx_csr_pcg_jacobi_cpu(it, n, data.numel(), _p(data), _p(indices), _p(indptr),
                                          _p(b), _p(x0), _p(inv_diag), _p(x), rtol, atol, maxiter,
                                          ctypes.byref(res))
    else:
        pp = plan.ptr if plan else None
        if inv_diag is None:
            st = L.msx_csr_cg(it, n, data.numel(), _p(data), _p(indices), _p(indptr), _p(b),
                              _p(x0), _p(x), rtol, atol, maxiter, pp, ctypes.byref(res), _stream())
        else:
            st = L.msx_csr_pcg_jacobi(it, n, data.numel(), _p(data), _p(indices), _p(indptr),
                                      _p(b), _p(x0), _p(inv_diag), _p(x), rtol, atol, maxiter, pp,
                                      ctypes.byref(res), _stream())
    _check(st, "msx_csr_cg")
    return x, res.info, res.residual, res.iterations


def krylov(kind, data, indices, indptr, b, x0=None, *, rtol=1e-5, atol=0.0, maxiter=None,
           shift=0.0, plan=None, inv_diag=None):
    """(x, info, residual, iterations) through msx_csr_bicgstab[_cpu]
    (kind "bicgstab") or msx_csr_minres[_cpu] (kind "minres"); with
    `inv_diag`, their Jacobi-preconditioned entry points (*_jacobi)."""
    n = b.numel()
    x0 = torch.zeros_like(b) if x0 is None else x0
    x = torch.empty_like(b)
    maxiter = 10 * n if maxiter is None else maxiter
    res = SolverResult()
    it = IT[indices.dtype]
    L = lib()
    pre = () if inv_diag is None else (_p(inv_diag),)
    if inv_diag is not None:
        kind = f"{kind}_jacobi"
    head = (it, n, data.numel(), _p(data), _p(indices), _p(indptr), _p(b), _p(x0), *pre, _p(x),
            rtol, atol, maxiter)
    extra = (shift,) if kind.startswith("minres") else ()
    if b.device.type == "cpu":
        st = getattr(L, f"msx_csr_{kind}_cpu")(*head, *extra, ctypes.byref(res))
    else:
        st = getattr(L, f"msx_csr_{kind}")(*head, *extra, plan.ptr if plan else None,
                                            ctypes.byref(res), _stream())
    _check(st, f"msx_csr_{kind}")
    return x, res.info, res.residual, res.iterations


def gmres(data, indices, indptr, b, x0=None, *, rtol=1e-5, atol=0.0, restart=None, maxiter=None,
          plan=None, inv_diag=None):
    """(x, info, residual, iterations) through msx_csr_gmres[_cpu]; with
    `inv_diag`, msx_csr_gmres_jacobi[_cpu]."""
    n = b.numel()
    x0 = torch.zeros_like(b) if x0 is None else x0
    x = torch.empty_like(b)
    restart = min(20, n) if restart is None else restart
    maxiter = 10 * n if maxiter is None else maxiter
    res = SolverResult()
    pre = () if inv_diag is None else (_p(inv_diag),)
    name = "msx_csr_gmres" if inv_diag is None else "msx_csr_gmres_jacobi"
    head = (IT[indices.dtype], n, data.numel(), _p(data), _p(indices), _p(indptr), _p(b), _p(x0),
            *pre, _p(x), rtol, atol, restart, maxiter)
    L = lib()
    if b.device.type == "cpu":
        st = getattr(L, f"{name}_cpu")(*head, ctypes.byref(res))
    else:
        st = getattr(L, name)(*head, plan.ptr if plan else None, ctypes.byref(res), _stream())
    _check(st, name)
    return x, res.info, res.residual, res.iterations
