"""Dispatch shim to the native module (reference: mlx_sparse/_native.py:179-189,
286-296).

The reference routes to ``_ext`` or, when the extension is missing, to a
NumPy fallback.  Here there is no fallback: a missing extension raises, so a
result always comes from the HIP kernels (GPU operands) or the native CPU
path (``use_cpu()``).
"""

from __future__ import annotations

import torch

from mlx_sparse._ext_loader import extension
from mlx_sparse._typing import Shape2D


def csr_matvec(data, indices, indptr, x, shape: Shape2D, plan=None) -> torch.Tensor:
    return extension().csr_matvec(data, indices, indptr, x, shape[0], shape[1], plan=plan)


def csr_matmul(data, indices, indptr, rhs, shape: Shape2D, plan=None) -> torch.Tensor:
    return extension().csr_matmul(data, indices, indptr, rhs, shape[0], shape[1], plan=plan)


def csr_batched_matvec(data, indices, indptr, rhs, shape: Shape2D) -> torch.Tensor:
    """(reference: mlx_sparse/_native.py:218-228)"""
    return extension().csr_batched_matvec(data, indices, indptr, rhs, shape[0], shape[1])


def csr_batched_matmul(data, indices, indptr, rhs, shape: Shape2D) -> torch.Tensor:
    """(reference: mlx_sparse/_native.py:325-335)"""
    return extension().csr_batched_matmul(data, indices, indptr, rhs, shape[0], shape[1])


def csr_transpose(data, indices, indptr, shape: Shape2D):
    """CSR buffers of A^T, shape (n_cols, n_rows) (reference:
    mlx_sparse/_native.py:464-473)."""
    return tuple(extension().csr_transpose(data, indices, indptr, shape[0], shape[1]))


def csr_transpose_positions(indices, indptr, shape: Shape2D):
    """(t_pos, t_indices, t_indptr): the structure of A^T and, per entry, the
    position of A it holds (int32; -1 for dropped values).  GPU only."""
    return tuple(extension().csr_transpose_positions(indices, indptr, shape[0], shape[1]))


def csr_transpose_values(data, positions, conjugate: bool, out) -> None:
    """out[i] = data[positions[i]] (conjugated on request), in place.  GPU only."""
    extension().csr_transpose_values(data, positions, conjugate, out)


def csr_transpose_layout(positions, like):
    """(slot1, src1, slot2): the layout of the two-pass regather of a
    transpose's values (dtype of ``like``), from its positions."""
    return tuple(extension().csr_transpose_layout(positions, like))


def csr_transpose_values_layout(data, layout, conjugate: bool, scratch, out) -> None:
    """``out`` = the regathered values through ``layout`` (``scratch``: as
    many values as ``data``, overwritten)."""
    slot1, src1, slot2 = layout
    extension().csr_transpose_values_layout(data, slot1, src1, slot2, conjugate, scratch, out)


def csr_matvec_transpose(data, indices, indptr, x, shape: Shape2D) -> torch.Tensor:
    """A^T x, without conjugation (reference: mlx_sparse/_native.py:260-270)."""
    return extension().csr_matvec_transpose(data, indices, indptr, x, shape[0], shape[1])


def csr_matmul_transpose(data, indices, indptr, rhs, shape: Shape2D) -> torch.Tensor:
    """A^T X, without conjugation (reference: mlx_sparse/_native.py:367-377)."""
    return extension().csr_matmul_transpose(data, indices, indptr, rhs, shape[0], shape[1])


def csr_matvec_data_vjp(indices, indptr, x, cotangent, shape: Shape2D, plan=None) -> torch.Tensor:
    """cot[row(p)] * x[col(p)] per stored value (reference:
    src/sparse/csr_matvec_data_vjp/csr_matvec_data_vjp.cpp); ``plan``: the
    matrix's GPU plan, whose panel layout (if any) serves the gather of x."""
    return extension().csr_matvec_data_vjp(indices, indptr, x, cotangent, shape[0], shape[1],
                                           plan=plan)


def csr_matmul_data_vjp(indices, indptr, rhs, cotangent, shape: Shape2D) -> torch.Tensor:
    """sum_q cot[row(p), q] * X[col(p), q] per stored value (reference:
    src/sparse/csr_matmul_data_vjp/csr_matmul_data_vjp.cpp)."""
    return extension().csr_matmul_data_vjp(indices, indptr, rhs, cotangent, shape[0], shape[1])


def csr_cg(data, indices, indptr, b, x0, shape: Shape2D, *, rtol: float, atol: float,
           maxiter: int, plan=None):
    """(x, info, residual, iterations) (reference: mlx_sparse/_native.py:883-905)."""
    return extension().csr_cg(data, indices, indptr, b, x0, shape[0], shape[1], rtol, atol,
                              maxiter, plan=plan)


def csr_pcg_jacobi(data, indices, indptr, b, x0, inv_diag, shape: Shape2D, *, rtol: float,
                   atol: float, maxiter: int, plan=None):
    """(x, info, residual, iterations) (reference: mlx_sparse/_native.py:1139-1166)."""
    return extension().csr_pcg_jacobi(data, indices, indptr, b, x0, inv_diag, shape[0], shape[1],
                                      rtol, atol, maxiter, plan=plan)


def csr_bicgstab(data, indices, indptr, b, x0, shape: Shape2D, *, rtol: float, atol: float,
                 maxiter: int, plan=None):
    """(x, info, residual, iterations) (reference: mlx_sparse/_native.py csr_bicgstab)."""
    return extension().csr_bicgstab(data, indices, indptr, b, x0, shape[0], shape[1], rtol, atol,
                                    maxiter, plan=plan)


def csr_bicgstab_jacobi(data, indices, indptr, b, x0, inv_diag, shape: Shape2D, *, rtol: float,
                        atol: float, maxiter: int, plan=None):
    """(x, info, residual, iterations) of Jacobi-preconditioned BiCGSTAB
    (reference: mlx_sparse/_native.py csr_bicgstab_jacobi)."""
    return extension().csr_bicgstab_jacobi(data, indices, indptr, b, x0, inv_diag, shape[0],
                                           shape[1], rtol, atol, maxiter, plan=plan)


def csr_minres(data, indices, indptr, b, x0, shape: Shape2D, *, rtol: float, atol: float,
               maxiter: int, shift: float = 0.0, plan=None):
    """(x, info, residual, iterations) of (A - shift I) x = b (reference:
    mlx_sparse/_native.py csr_minres)."""
    return extension().csr_minres(data, indices, indptr, b, x0, shape[0], shape[1], rtol, atol,
                                  maxiter, shift, plan=plan)


def csr_minres_jacobi(data, indices, indptr, b, x0, inv_diag, shape: Shape2D, *, rtol: float,
                      atol: float, maxiter: int, shift: float = 0.0, plan=None):
    """(x, info, residual, iterations) of Jacobi-preconditioned MINRES on
    (A - shift I) x = b (reference: mlx_sparse/_native.py csr_minres_jacobi)."""
    return extension().csr_minres_jacobi(data, indices, indptr, b, x0, inv_diag, shape[0],
                                         shape[1], rtol, atol, maxiter, shift, plan=plan)


def csr_gmres(data, indices, indptr, b, x0, shape: Shape2D, *, rtol: float, atol: float,
              restart: int, maxiter: int, plan=None):
    """(x, info, residual, iterations) of restarted GMRES (reference:
    mlx_sparse/_native.py:1505-1530 csr_gmres)."""
    return extension().csr_gmres(data, indices, indptr, b, x0, shape[0], shape[1], rtol, atol,
                                 restart, maxiter, plan=plan)


def csr_gmres_jacobi(data, indices, indptr, b, x0, inv_diag, shape: Shape2D, *, rtol: float,
                     atol: float, restart: int, maxiter: int, plan=None):
    """(x, info, residual, iterations) of Jacobi-preconditioned restarted
    GMRES (reference: mlx_sparse/_native.py csr_gmres_jacobi)."""
    return extension().csr_gmres_jacobi(data, indices, indptr, b, x0, inv_diag, shape[0],
                                        shape[1], rtol, atol, restart, maxiter, plan=plan)


def csr_plan(indptr, n_rows: int, nnz: int, block_nnz: int = 0, *, data=None, indices=None,
             n_cols: int = -1, slice_mode: int = 0):
    """Row-block plan; with ``data``/``indices`` a plan bound to the matrix,
    which may hold a reordered copy for scattered gathers (slice_mode 0 auto,
    1 off, 2 XCD column slices, 3 LDS column panels)."""
    return extension().csr_plan(indptr, n_rows, nnz, block_nnz, data=data, indices=indices,
                                n_cols=n_cols, slice_mode=slice_mode)
