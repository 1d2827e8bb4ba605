"""CPU oracle for the CSR sparse x dense path - TEST INFRASTRUCTURE ONLY.

ctypes front end of ``csr_oracle.c`` (a plain-C restatement of mlx-sparse's
CPU kernels, reference: src/sparse/csr_matvec/csr_matvec.cpp:79-168,
src/sparse/csr_matmul/csr_matmul.cpp:83-222, src/common/common.h:52-79,
src/common/cpu_parallel.cpp:46-253, and the adjoint side:
src/sparse/csr_transpose, csr_matvec_transpose, csr_matmul_transpose,
csr_matvec_data_vjp, csr_matmul_data_vjp).  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import
this module, always as the checker or the timed CPU baseline, never as the
product path.

Value arrays are numpy arrays of the storage type: float32, float16,
complex64, and bfloat16 as raw ``uint16`` bit patterns (numpy has no
bfloat16).  Pass ``vtype`` explicitly for bfloat16.

Parity status of each function (the checks live in tests/test_oracle_*.py):

- ``csr_matvec``/``csr_matmul`` float32: pinned (reference KATs, SciPy,
  SuiteSparse fixtures, closed forms, float64 brute force).
- float16/bfloat16: pinned to the rule "widen, multiply and sum in float32,
  round once (nearest even)"; the rounding functions are pinned against
  numpy float16 and torch bfloat16 casts.  MLX's own rounding is un-vendored.
- complex64: pinned against numpy complex products and the split into real
  SpMVs; the bit pattern of MLX's complex product is un-vendored.
- ``cpu_ranges``/``cpu_worker_count``: pinned against a naive re-derivation
  and environment cases.
- ``csr_transpose``: pinned against SciPy's ``tocsc`` (same stable order)
  and a dense transpose.
- ``csr_transpose_product``: float32 pinned against float64 brute force, the
  adjoint identity <A x, y> = <x, A^T y>, single-product closed forms and the
  transpose-then-SpMV route on matrices whose columns hold one value; the
  W-worker partial order pinned on a case where it changes the rounding.
- ``csr_data_vjp``: pinned against finite differences of the dense product
  (exact for float32 on small integers) and the single-product rule.
- ``csr_cg`` / ``csr_pcg_jacobi``: pinned against a dense float64 solve
  (SPD systems), the CG closed form on a diagonal system (one iteration per
  distinct eigenvalue), SciPy's ``cg`` iteration counts on the same
  systems, and the status rules (zero right-hand side, maxiter = 0,
  non-finite input, indefinite matrix, non-positive preconditioner).
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "libcsr_oracle.so"

VTYPES = {"float32": 0, "float16": 1, "bfloat16": 2, "complex64": 3}
ITYPES = {np.dtype(np.int32): 0, np.dtype(np.int64): 1}
_STORAGE = {
    "float32": np.dtype(np.float32),
    "float16": np.dtype(np.float16),
    "bfloat16": np.dtype(np.uint16),
    "complex64": np.dtype(np.complex64),
}

_lib = None


def build() -> Path:
    """Compile the oracle with its Makefile (gcc, -O3, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(_LIB_PATH))
        vp, i64, ci = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        _lib.oracle_csr_matvec.argtypes = [ci, ci, i64, vp, vp, vp, vp, vp, ci]
        _lib.oracle_csr_matvec.restype = ci
        _lib.oracle_csr_matmul.argtypes = [ci, ci, i64, i64, vp, vp, vp, vp, vp, ci]
        _lib.oracle_csr_matmul.restype = ci
        _lib.oracle_cpu_ranges.argtypes = [vp, i64, ci, vp]
        _lib.oracle_cpu_ranges.restype = i64
        _lib.oracle_cpu_worker_count.argtypes = []
        _lib.oracle_cpu_worker_count.restype = ci
        _lib.oracle_narrow_array.argtypes = [ci, vp, vp, i64]
        _lib.oracle_narrow_array.restype = None
        _lib.oracle_widen_array.argtypes = [ci, vp, vp, i64]
        _lib.oracle_widen_array.restype = None
        _lib.oracle_csr_transpose_product.argtypes = [ci, ci, i64, i64, i64, vp, vp, vp, vp, vp,
                                                      ci]
        _lib.oracle_csr_transpose_product.restype = ci
        _lib.oracle_csr_transpose.argtypes = [ci, ci, i64, i64, vp, vp, vp, vp, vp, vp]
        _lib.oracle_csr_transpose.restype = ci
        _lib.oracle_csr_data_vjp.argtypes = [ci, ci, i64, i64, i64, ci, vp, vp, vp, vp, vp]
        _lib.oracle_csr_data_vjp.restype = ci
        f32 = ctypes.c_float
        _lib.oracle_csr_cg.argtypes = [ci, i64, vp, vp, vp, vp, vp, vp, f32, f32, i64, vp, vp, vp]
        _lib.oracle_csr_cg.restype = ci
        _lib.oracle_csr_pcg_jacobi.argtypes = [ci, i64, vp, vp, vp, vp, vp, vp, vp, f32, f32, i64,
                                               vp, vp, vp]
        _lib.oracle_csr_pcg_jacobi.restype = ci
        _lib.oracle_csr_bicgstab.argtypes = [ci, i64, vp, vp, vp, vp, vp, vp, f32, f32, i64, vp,
                                             vp, vp]
        _lib.oracle_csr_bicgstab.restype = ci
        _lib.oracle_csr_bicgstab_jacobi.argtypes = [ci, i64, vp, vp, vp, vp, vp, vp, vp, f32, f32,
                                                    i64, vp, vp, vp]
        _lib.oracle_csr_bicgstab_jacobi.restype = ci
        _lib.oracle_csr_minres.argtypes = [ci, i64, vp, vp, vp, vp, vp, vp, f32, f32, i64, f32,
                                           vp, vp, vp]
        _lib.oracle_csr_minres.restype = ci
        _lib.oracle_csr_minres_jacobi.argtypes = [ci, i64, vp, vp, vp, vp, vp, vp, vp, f32, f32,
                                                  i64, f32, vp, vp, vp]
        _lib.oracle_csr_minres_jacobi.restype = ci
        _lib.oracle_csr_arnoldi.argtypes = [ci, i64, vp, vp, vp, vp, i64, vp, vp, vp]
        _lib.oracle_csr_arnoldi.restype = ci
        _lib.oracle_csr_gmres.argtypes = [ci, i64, vp, vp, vp, vp, vp, vp, f32, f32, i64, i64,
                                          vp, vp, vp]
        _lib.oracle_csr_gmres.restype = ci
        _lib.oracle_csr_arnoldi_jacobi.argtypes = [ci, i64, vp, vp, vp, vp, vp, i64, vp, vp, vp]
        _lib.oracle_csr_arnoldi_jacobi.restype = ci
        _lib.oracle_csr_gmres_jacobi.argtypes = [ci, i64, vp, vp, vp, vp, vp, vp, vp, f32, f32,
                                                 i64, i64, vp, vp, vp]
        _lib.oracle_csr_gmres_jacobi.restype = ci
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def _vtype_of(arr: np.ndarray, vtype: str | None) -> str:
    if vtype is not None:
        return vtype
    for name, dt in _STORAGE.items():
        if arr.dtype == dt and name != "bfloat16":
            return name
    raise TypeError(f"oracle: unsupported value dtype {arr.dtype}")


def _prep(data, indices, indptr, vtype):
    vt = _vtype_of(np.asarray(data), vtype)
    data = np.ascontiguousarray(data, dtype=_STORAGE[vt])
    indices = np.ascontiguousarray(indices)
    indptr = np.ascontiguousarray(indptr)
    if indices.dtype != indptr.dtype or indices.dtype not in ITYPES:
        raise TypeError("oracle: indices/indptr must share int32 or int64")
    return vt, data, indices, indptr


def csr_matvec(data, indices, indptr, x, n_rows: int, *, vtype: str | None = None,
               n_threads: int = 1) -> np.ndarray:
    """Sequential-order CSR SpMV (reference csr_matvec.cpp:79-168)."""
    vt, data, indices, indptr = _prep(data, indices, indptr, vtype)
    x = np.ascontiguousarray(x, dtype=_STORAGE[vt])
    y = np.empty(n_rows, dtype=_STORAGE[vt])
    rc = lib().oracle_csr_matvec(VTYPES[vt], ITYPES[indices.dtype], n_rows, _ptr(data),
                                 _ptr(indices), _ptr(indptr), _ptr(x), _ptr(y), n_threads)
    if rc != 0:
        raise MemoryError("oracle_csr_matvec failed")
    return y


def csr_matmul(data, indices, indptr, X, n_rows: int, *, vtype: str | None = None,
               n_threads: int = 1) -> np.ndarray:
    """Sequential-order CSR SpMM with row-major X (reference csr_matmul.cpp:83-222)."""
    vt, data, indices, indptr = _prep(data, indices, indptr, vtype)
    X = np.ascontiguousarray(X, dtype=_STORAGE[vt])
    if X.ndim != 2:
        raise ValueError("oracle: X must be rank-2")
    k = X.shape[1]
    Y = np.empty((n_rows, k), dtype=_STORAGE[vt])
    rc = lib().oracle_csr_matmul(VTYPES[vt], ITYPES[indices.dtype], n_rows, k, _ptr(data),
                                 _ptr(indices), _ptr(indptr), _ptr(X), _ptr(Y), n_threads)
    if rc != 0:
        raise MemoryError("oracle_csr_matmul failed")
    return Y


def csr_transpose_product(data, indices, indptr, X, n_rows: int, n_cols: int, *,
                          vtype: str | None = None, n_threads: int = 1) -> np.ndarray:
    """A^T x (X rank 1) or A^T X (rank 2, row-major): one worker sums every
    output from zero over the rows in order; W workers keep one partial
    output per row range (ranges by row length) and add the partials from
    zero in range order (reference csr_matvec_transpose.cpp:89-153,
    csr_matmul_transpose.cpp:94-159).  Complex values are not conjugated."""
    vt, data, indices, indptr = _prep(data, indices, indptr, vtype)
    X = np.ascontiguousarray(X, dtype=_STORAGE[vt])
    k = 1 if X.ndim == 1 else X.shape[1]
    shape = (n_cols,) if X.ndim == 1 else (n_cols, k)
    Y = np.empty(shape, dtype=_STORAGE[vt])
    rc = lib().oracle_csr_transpose_product(VTYPES[vt], ITYPES[indices.dtype], n_rows, n_cols,
                                            k, _ptr(data), _ptr(indices), _ptr(indptr), _ptr(X),
                                            _ptr(Y), n_threads)
    if rc != 0:
        raise MemoryError("oracle_csr_transpose_product failed")
    return Y


def csr_transpose(data, indices, indptr, n_rows: int, n_cols: int, *,
                  vtype: str | None = None):
    """CSR of A^T by counting sort: column counts, prefix sums, then the
    stored values scattered in row order (reference
    csr_transpose.cpp, csr_transpose_cpu_impl).  Returns (data, indices,
    indptr) of the (n_cols, n_rows) transpose."""
    vt, data, indices, indptr = _prep(data, indices, indptr, vtype)
    nnz = int(indptr[n_rows]) if n_rows > 0 else 0
    t_data = np.empty(max(nnz, 0), dtype=_STORAGE[vt])
    t_indices = np.empty(max(nnz, 0), dtype=indices.dtype)
    t_indptr = np.empty(n_cols + 1, dtype=indices.dtype)
    rc = lib().oracle_csr_transpose(VTYPES[vt], ITYPES[indices.dtype], n_rows, n_cols,
                                    _ptr(data), _ptr(indices), _ptr(indptr), _ptr(t_data),
                                    _ptr(t_indices), _ptr(t_indptr))
    if rc != 0:
        raise MemoryError("oracle_csr_transpose failed")
    end = int(t_indptr[n_cols])
    return t_data[:end], t_indices[:end], t_indptr


def csr_data_vjp(indices, indptr, X, cot, n_rows: int, n_cols: int, nnz: int, *,
                 vtype: str | None = None) -> np.ndarray:
    """Gradient of the stored values.  X rank 1 (SpMV): g[p] = cot[row] *
    x[col], one product (reference csr_matvec_data_vjp.cpp).  X rank 2:
    g[p] = sum_q cot[row, q] * X[col, q] from zero (csr_matmul_data_vjp.cpp).
    No conjugation: complex callers pass conj(x)."""
    X = np.asarray(X)
    vt = _vtype_of(X, vtype)
    indices = np.ascontiguousarray(indices)
    indptr = np.ascontiguousarray(indptr)
    X = np.ascontiguousarray(X, dtype=_STORAGE[vt])
    cot = np.ascontiguousarray(cot, dtype=_STORAGE[vt])
    single = 1 if X.ndim == 1 else 0
    k = 1 if X.ndim == 1 else X.shape[1]
    out = np.zeros(nnz, dtype=_STORAGE[vt])
    rc = lib().oracle_csr_data_vjp(VTYPES[vt], ITYPES[indices.dtype], n_rows, n_cols, k, single,
                                   _ptr(indices), _ptr(indptr), _ptr(X), _ptr(cot), _ptr(out))
    if rc != 0:
        raise MemoryError("oracle_csr_data_vjp failed")
    return out


def _solver_inputs(data, indices, indptr, b, x0):
    data = np.ascontiguousarray(data, dtype=np.float32)
    indices = np.ascontiguousarray(indices)
    indptr = np.ascontiguousarray(indptr)
    if indices.dtype != indptr.dtype or indices.dtype not in ITYPES:
        raise TypeError("oracle: indices/indptr must share int32 or int64")
    b = np.ascontiguousarray(b, dtype=np.float32)
    n = b.shape[0]
    x0 = np.zeros(n, np.float32) if x0 is None else np.ascontiguousarray(x0, dtype=np.float32)
    return data, indices, indptr, b, x0, n


def csr_cg(data, indices, indptr, b, x0=None, *, rtol: float = 1e-5, atol: float = 0.0,
           maxiter: int | None = None):
    """Conjugate gradients on a square float32 CSR matrix (reference
    src/linalg/cg/cg.cpp:75-246).  Returns (x, info, residual, iterations)."""
    data, indices, indptr, b, x0, n = _solver_inputs(data, indices, indptr, b, x0)
    maxiter = 10 * n if maxiter is None else int(maxiter)
    x = np.empty(n, np.float32)
    info, res, its = ctypes.c_int32(), ctypes.c_float(), ctypes.c_int32()
    rc = lib().oracle_csr_cg(ITYPES[indices.dtype], n, _ptr(data), _ptr(indices), _ptr(indptr),
                             _ptr(b), _ptr(x0), _ptr(x), rtol, atol, maxiter, ctypes.addressof(info),
                             ctypes.addressof(res), ctypes.addressof(its))
    if rc != 0:
        raise MemoryError("oracle_csr_cg failed")
    return x, info.value, res.value, its.value


def csr_pcg_jacobi(data, indices, indptr, b, inv_diag, x0=None, *, rtol: float = 1e-5,
                   atol: float = 0.0, maxiter: int | None = None):
    """Jacobi-preconditioned CG (reference src/preconditioners/pcg/pcg.cpp:71-236).
    Returns (x, info, residual, iterations)."""
    data, indices, indptr, b, x0, n = _solver_inputs(data, indices, indptr, b, x0)
    inv_diag = np.ascontiguousarray(inv_diag, dtype=np.float32)
    maxiter = 10 * n if maxiter is None else int(maxiter)
    x = np.empty(n, np.float32)
    info, res, its = ctypes.c_int32(), ctypes.c_float(), ctypes.c_int32()
    rc = lib().oracle_csr_pcg_jacobi(ITYPES[indices.dtype], n, _ptr(data), _ptr(indices),
                                     _ptr(indptr), _ptr(b), _ptr(x0), _ptr(inv_diag), _ptr(x),
                                     rtol, atol, maxiter, ctypes.addressof(info),
                                     ctypes.addressof(res), ctypes.addressof(its))
    if rc != 0:
        raise MemoryError("oracle_csr_pcg_jacobi failed")
    return x, info.value, res.value, its.value


def csr_bicgstab(data, indices, indptr, b, x0=None, *, rtol: float = 1e-5, atol: float = 0.0,
                 maxiter: int | None = None):
    """BiCGSTAB on a square float32 CSR matrix (reference
    src/linalg/bicgstab/bicgstab.cpp:80-362).  Returns (x, info, residual,
    iterations)."""
    data, indices, indptr, b, x0, n = _solver_inputs(data, indices, indptr, b, x0)
    maxiter = 10 * n if maxiter is None else int(maxiter)
    x = np.empty(n, np.float32)
    info, res, its = ctypes.c_int32(), ctypes.c_float(), ctypes.c_int32()
    rc = lib().oracle_csr_bicgstab(ITYPES[indices.dtype], n, _ptr(data), _ptr(indices),
                                   _ptr(indptr), _ptr(b), _ptr(x0), _ptr(x), rtol, atol, maxiter,
                                   ctypes.addressof(info), ctypes.addressof(res),
                                   ctypes.addressof(its))
    if rc != 0:
        raise MemoryError("oracle_csr_bicgstab failed")
    return x, info.value, res.value, its.value


def csr_bicgstab_jacobi(data, indices, indptr, b, inv_diag, x0=None, *, rtol: float = 1e-5,
                        atol: float = 0.0, maxiter: int | None = None):
    """BiCGSTAB with the Jacobi preconditioner M = diag(inv_diag) (reference
    src/preconditioners/bicgstab/bicgstab.cpp:140-521,
    left_preconditioned_bicgstab_host with csr_bicgstab_jacobi_cpu_impl's
    apply).  Returns (x, info, residual, iterations)."""
    data, indices, indptr, b, x0, n = _solver_inputs(data, indices, indptr, b, x0)
    inv_diag = np.ascontiguousarray(inv_diag, np.float32)
    assert inv_diag.shape == (n,)
    maxiter = 10 * n if maxiter is None else int(maxiter)
    x = np.empty(n, np.float32)
    info, res, its = ctypes.c_int32(), ctypes.c_float(), ctypes.c_int32()
    rc = lib().oracle_csr_bicgstab_jacobi(ITYPES[indices.dtype], n, _ptr(data), _ptr(indices),
                                          _ptr(indptr), _ptr(b), _ptr(x0), _ptr(inv_diag),
                                          _ptr(x), rtol, atol, maxiter, ctypes.addressof(info),
                                          ctypes.addressof(res), ctypes.addressof(its))
    if rc != 0:
        raise MemoryError("oracle_csr_bicgstab_jacobi failed")
    return x, info.value, res.value, its.value


def csr_minres(data, indices, indptr, b, x0=None, *, rtol: float = 1e-5, atol: float = 0.0,
               maxiter: int | None = None, shift: float = 0.0):
    """MINRES on (A - shift I) x = b, A square symmetric float32 CSR
    (reference src/linalg/minres/minres.cpp:68-312).  Returns (x, info,
    residual, iterations)."""
    data, indices, indptr, b, x0, n = _solver_inputs(data, indices, indptr, b, x0)
    maxiter = 10 * n if maxiter is None else int(maxiter)
    x = np.empty(n, np.float32)
    info, res, its = ctypes.c_int32(), ctypes.c_float(), ctypes.c_int32()
    rc = lib().oracle_csr_minres(ITYPES[indices.dtype], n, _ptr(data), _ptr(indices),
                                 _ptr(indptr), _ptr(b), _ptr(x0), _ptr(x), rtol, atol, maxiter,
                                 shift, ctypes.addressof(info), ctypes.addressof(res),
                                 ctypes.addressof(its))
    if rc != 0:
        raise MemoryError("oracle_csr_minres failed")
    return x, info.value, res.value, its.value


def csr_minres_jacobi(data, indices, indptr, b, inv_diag, x0=None, *, rtol: float = 1e-5,
                      atol: float = 0.0, maxiter: int | None = None, shift: float = 0.0):
    """MINRES with the Jacobi preconditioner M = diag(inv_diag) on
    (A - shift I) x = b (reference src/preconditioners/minres/minres.cpp:93-330,
    csr_minres_jacobi_cpu_impl).  Returns (x, info, residual, iterations)."""
    data, indices, indptr, b, x0, n = _solver_inputs(data, indices, indptr, b, x0)
    inv_diag = np.ascontiguousarray(inv_diag, np.float32)
    assert inv_diag.shape == (n,)
    maxiter = 10 * n if maxiter is None else int(maxiter)
    x = np.empty(n, np.float32)
    info, res, its = ctypes.c_int32(), ctypes.c_float(), ctypes.c_int32()
    rc = lib().oracle_csr_minres_jacobi(ITYPES[indices.dtype], n, _ptr(data), _ptr(indices),
                                        _ptr(indptr), _ptr(b), _ptr(x0), _ptr(inv_diag), _ptr(x),
                                        rtol, atol, maxiter, shift, ctypes.addressof(info),
                                        ctypes.addressof(res), ctypes.addressof(its))
    if rc != 0:
        raise MemoryError("oracle_csr_minres_jacobi failed")
    return x, info.value, res.value, its.value


def csr_arnoldi(data, indices, indptr, v0, k: int):
    """k Arnoldi steps of a square float32 CSR matrix from v0 (reference
    src/linalg/arnoldi/arnoldi.cpp:79-159).  Returns (h of shape (k+1, k),
    basis of shape (n, k+1), used)."""
    data, indices, indptr, v0, _, n = _solver_inputs(data, indices, indptr, v0, None)
    h = np.empty((k + 1, k), np.float32)
    basis = np.empty((n, k + 1), np.float32)
    used = ctypes.c_int32()
    rc = lib().oracle_csr_arnoldi(ITYPES[indices.dtype], n, _ptr(data), _ptr(indices),
                                  _ptr(indptr), _ptr(v0), k, _ptr(h), _ptr(basis),
                                  ctypes.addressof(used))
    if rc != 0:
        raise MemoryError("oracle_csr_arnoldi failed")
    return h, basis, used.value


def csr_gmres(data, indices, indptr, b, x0=None, *, rtol: float = 1e-5, atol: float = 0.0,
              restart: int | None = None, maxiter: int | None = None):
    """Restarted GMRES on a square float32 CSR matrix (reference
    src/linalg/gmres/gmres.cpp:58-220).  ``restart`` defaults to min(20, n),
    ``maxiter`` (Arnoldi steps over all cycles) to 10 n.  Returns (x, info,
    residual, iterations)."""
    data, indices, indptr, b, x0, n = _solver_inputs(data, indices, indptr, b, x0)
    restart = min(20, n) if restart is None else int(restart)
    maxiter = 10 * n if maxiter is None else int(maxiter)
    x = np.empty(n, np.float32)
    info, res, its = ctypes.c_int32(), ctypes.c_float(), ctypes.c_int32()
    rc = lib().oracle_csr_gmres(ITYPES[indices.dtype], n, _ptr(data), _ptr(indices),
                                _ptr(indptr), _ptr(b), _ptr(x0), _ptr(x), rtol, atol, restart,
                                maxiter, ctypes.addressof(info), ctypes.addressof(res),
                                ctypes.addressof(its))
    if rc != 0:
        raise MemoryError("oracle_csr_gmres failed")
    return x, info.value, res.value, its.value


def csr_arnoldi_jacobi(data, indices, indptr, inv_diag, v0, k: int):
    """k Jacobi Arnoldi steps (the basis of M A, M = diag(inv_diag);
    reference src/preconditioners/gmres/gmres.cpp:342-447).  Returns (h,
    basis, used) as csr_arnoldi."""
    data, indices, indptr, v0, _, n = _solver_inputs(data, indices, indptr, v0, None)
    inv_diag = np.ascontiguousarray(inv_diag, np.float32)
    assert inv_diag.shape == (n,)
    h = np.empty((k + 1, k), np.float32)
    basis = np.empty((n, k + 1), np.float32)
    used = ctypes.c_int32()
    rc = lib().oracle_csr_arnoldi_jacobi(ITYPES[indices.dtype], n, _ptr(data), _ptr(indices),
                                         _ptr(indptr), _ptr(inv_diag), _ptr(v0), k, _ptr(h),
                                         _ptr(basis), ctypes.addressof(used))
    if rc != 0:
        raise MemoryError("oracle_csr_arnoldi_jacobi failed")
    return h, basis, used.value


def csr_gmres_jacobi(data, indices, indptr, b, inv_diag, x0=None, *, rtol: float = 1e-5,
                     atol: float = 0.0, restart: int | None = None,
                     maxiter: int | None = None):
    """Restarted GMRES with the Jacobi preconditioner M = diag(inv_diag)
    (reference src/preconditioners/gmres/gmres.cpp:572-748).  Returns (x,
    info, residual, iterations)."""
    data, indices, indptr, b, x0, n = _solver_inputs(data, indices, indptr, b, x0)
    inv_diag = np.ascontiguousarray(inv_diag, np.float32)
    assert inv_diag.shape == (n,)
    restart = min(20, n) if restart is None else int(restart)
    maxiter = 10 * n if maxiter is None else int(maxiter)
    x = np.empty(n, np.float32)
    info, res, its = ctypes.c_int32(), ctypes.c_float(), ctypes.c_int32()
    rc = lib().oracle_csr_gmres_jacobi(ITYPES[indices.dtype], n, _ptr(data), _ptr(indices),
                                       _ptr(indptr), _ptr(b), _ptr(x0), _ptr(inv_diag), _ptr(x),
                                       rtol, atol, restart, maxiter, ctypes.addressof(info),
                                       ctypes.addressof(res), ctypes.addressof(its))
    if rc != 0:
        raise MemoryError("oracle_csr_gmres_jacobi failed")
    return x, info.value, res.value, its.value


def cpu_ranges(work, parts: int) -> list[tuple[int, int]]:
    """cpu_ranges_for_output_work (reference cpu_parallel.h:134-164)."""
    work = np.ascontiguousarray(work, dtype=np.int64)
    out = np.empty(2 * max(parts, 1), dtype=np.int64)
    m = lib().oracle_cpu_ranges(_ptr(work), work.size, parts, _ptr(out))
    if m < 0:
        raise MemoryError("oracle_cpu_ranges failed")
    return [(int(out[2 * i]), int(out[2 * i + 1])) for i in range(m)]


def cpu_worker_count() -> int:
    """configured_cpu_worker_count (reference cpu_parallel.cpp:97-135)."""
    return int(lib().oracle_cpu_worker_count())


def f32_to_bf16_bits(a) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().oracle_narrow_array(1, _ptr(a), _ptr(out), a.size)
    return out


def f32_to_f16_bits(a) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().oracle_narrow_array(0, _ptr(a), _ptr(out), a.size)
    return out


def bf16_bits_to_f32(a) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    out = np.empty(a.shape, dtype=np.float32)
    lib().oracle_widen_array(1, _ptr(a), _ptr(out), a.size)
    return out


def f16_bits_to_f32(a) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    out = np.empty(a.shape, dtype=np.float32)
    lib().oracle_widen_array(0, _ptr(a), _ptr(out), a.size)
    return out


def row_scale(data, indices, indptr, x, n_rows: int, *, vtype: str | None = None) -> np.ndarray:
    """Per-row sum of |a_ij * x_j| in float64, the scale of the parity tolerance."""
    vt = _vtype_of(np.asarray(data), vtype)
    d = np.asarray(data)
    xv = np.asarray(x)
    if vt == "bfloat16":
        d = bf16_bits_to_f32(d)
        xv = bf16_bits_to_f32(xv)
    d = np.abs(d.astype(np.complex128 if vt == "complex64" else np.float64))
    xv = np.abs(xv.astype(np.complex128 if vt == "complex64" else np.float64))
    indptr = np.asarray(indptr, dtype=np.int64)
    rows = np.repeat(np.arange(n_rows), np.diff(indptr))
    if xv.ndim == 1:
        terms = d * xv[np.asarray(indices, dtype=np.int64)]
        return np.bincount(rows, weights=terms, minlength=n_rows)
    terms = d[:, None] * xv[np.asarray(indices, dtype=np.int64)]
    out = np.zeros((n_rows, xv.shape[1]))
    np.add.at(out, rows, terms)
    return out


def row_exact(data, indices, indptr, x, n_rows: int, *, vtype: str | None = None) -> np.ndarray:
    """Per-row sum of a_ij * x_j in float64 / complex128: products of two
    binary16/bfloat16/binary32 values are exact in binary64, so only the
    float64 summation rounds (relative error ~ n * 2^-53)."""
    vt = _vtype_of(np.asarray(data), vtype)
    d, xv = np.asarray(data), np.asarray(x)
    if vt == "bfloat16":
        d, xv = bf16_bits_to_f32(d), bf16_bits_to_f32(xv)
    wide = np.complex128 if vt == "complex64" else np.float64
    d, xv = d.astype(wide), xv.astype(wide)
    indptr = np.asarray(indptr, dtype=np.int64)
    rows = np.repeat(np.arange(n_rows), np.diff(indptr))
    cols = np.asarray(indices, dtype=np.int64)
    if xv.ndim == 1:
        terms = d * xv[cols]
        if vt == "complex64":
            return (np.bincount(rows, weights=terms.real, minlength=n_rows)
                    + 1j * np.bincount(rows, weights=terms.imag, minlength=n_rows))
        return np.bincount(rows, weights=terms, minlength=n_rows)
    out = np.zeros((n_rows, xv.shape[1]), dtype=wide)
    np.add.at(out, rows, d[:, None] * xv[cols])
    return out


__all__ = [
    "VTYPES",
    "build",
    "lib",
    "csr_matvec",
    "csr_matmul",
    "cpu_ranges",
    "cpu_worker_count",
    "f32_to_bf16_bits",
    "f32_to_f16_bits",
    "bf16_bits_to_f32",
    "f16_bits_to_f32",
    "row_scale",
    "row_exact",
]
