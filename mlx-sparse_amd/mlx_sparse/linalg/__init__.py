"""Sparse iterative solvers on the path's SpMV (reference:
mlx_sparse/linalg/__init__.py): conjugate gradients (plain and
Jacobi-preconditioned), BiCGSTAB, MINRES and restarted GMRES, device-resident
on MI355X."""

from __future__ import annotations

from mlx_sparse.linalg import preconditioners
from mlx_sparse.linalg._info import SolverInfo
from mlx_sparse.linalg._iterative import bicgstab, cg, gmres, minres

__all__ = ["SolverInfo", "bicgstab", "cg", "gmres", "minres", "preconditioners"]
