"""Preconditioners the native CG accepts (reference:
mlx_sparse/linalg/preconditioners.py:78-293, 998-1150, 1546): identity,
explicit diagonal and Jacobi.  Each holds a float32 inverse diagonal (or
nothing, for the identity) on the selected device."""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from mlx_sparse._csr import CSRArray
from mlx_sparse._device import default_torch_device
from mlx_sparse._validation import ensure_array


@dataclass(frozen=True)
class IdentityPreconditioner:
    shape: tuple[int, int]
    kind: str = "identity"
    is_symmetric: bool = True

    def __call__(self, x):
        return x


@dataclass(frozen=True)
class DiagonalPreconditioner:
    inverse_diagonal: torch.Tensor
    shape: tuple[int, int]
    kind: str = "diagonal"
    is_symmetric: bool = True

    def __call__(self, x):
        return self.inverse_diagonal * x if x.ndim == 1 else self.inverse_diagonal[:, None] * x


@dataclass(frozen=True)
class JacobiPreconditioner(DiagonalPreconditioner):
    kind: str = "jacobi"
    omega: float = 1.0
    shift: float = 0.0


def _square(n: int) -> tuple[int, int]:
    return (int(n), int(n))


def _float32_vector(name: str, values) -> torch.Tensor:
    v = ensure_array(values, device=default_torch_device())
    if v.ndim != 1:
        raise ValueError(f"{name} must be rank-1, got shape {tuple(v.shape)}.")
    if v.is_complex():
        raise TypeError(f"{name} must be real.")
    return v.to(torch.float32).contiguous()


def identity(A_or_shape, *, dtype=None) -> IdentityPreconditioner:
    """The identity (no preconditioning)."""
    if dtype is not None and dtype != torch.float32:
        raise TypeError("identity preconditioners currently use float32 values.")
    shape = A_or_shape.shape if hasattr(A_or_shape, "shape") else tuple(A_or_shape)
    if len(shape) != 2 or shape[0] != shape[1]:
        raise ValueError(f"identity requires a square shape, got {shape}.")
    return IdentityPreconditioner(_square(shape[0]))


def diagonal(inv_diag_or_diag, *, inverse: bool = False, shape=None, dtype=None,
             zero_atol: float = 0.0) -> DiagonalPreconditioner:
    """Explicit diagonal inverse-apply preconditioner: ``inv_diag_or_diag`` is
    a diagonal (inverted here) or, with ``inverse=True``, the inverse itself."""
    values = _float32_vector("diagonal", inv_diag_or_diag)
    if not bool(torch.isfinite(values).all()):
        raise ValueError("diagonal must contain only finite values.")
    if dtype is not None and dtype != torch.float32:
        raise TypeError("diagonal preconditioners currently use float32 values.")
    pc_shape = _square(values.shape[0]) if shape is None else tuple(int(s) for s in shape)
    if len(pc_shape) != 2 or pc_shape[0] != pc_shape[1]:
        raise ValueError(f"diagonal requires a square shape, got {pc_shape}.")
    if values.shape[0] != pc_shape[0]:
        raise ValueError(f"diagonal has length {values.shape[0]}, expected {pc_shape[0]}.")
    if inverse:
        inv = values
    else:
        if zero_atol < 0.0:
            raise ValueError("zero_atol must be non-negative.")
        if bool((values.abs() <= zero_atol).any()):
            raise ValueError("diagonal contains zero or near-zero entries.")
        inv = 1.0 / values
    return DiagonalPreconditioner(inv, pc_shape)


def csr_diagonal(A: CSRArray, device=None) -> torch.Tensor:
    """Main diagonal of a CSR matrix, duplicates summed (float32)."""
    device = default_torch_device() if device is None else torch.device(device)
    data, indices, indptr = A.buffers(device)
    n_rows, n_cols = A.shape
    rows = torch.repeat_interleave(torch.arange(n_rows, device=device),
                                   (indptr[1:] - indptr[:-1]).to(torch.int64))
    on = rows == indices.to(torch.int64)
    out = torch.zeros(min(n_rows, n_cols), dtype=torch.float32, device=device)
    out.index_add_(0, rows[on], data[on].to(torch.float32))
    return out


def jacobi(A, *, omega: float = 1.0, shift: float = 0.0, zero_policy: str = "raise",
           zero_atol: float = 0.0, check: bool = False) -> JacobiPreconditioner:
    """Jacobi preconditioner ``omega / (diag(A) + shift)``."""
    if zero_policy not in {"raise", "unit"}:
        raise ValueError("zero_policy must be 'raise' or 'unit'.")
    for name, v in (("omega", omega), ("shift", shift)):
        if not math.isfinite(float(v)):
            raise ValueError(f"{name} must be finite.")
    if check and omega <= 0.0:
        raise ValueError("omega must be positive when check=True.")
    if not isinstance(A, CSRArray):
        raise TypeError("jacobi expects a CSRArray.")
    if A.shape[0] != A.shape[1]:
        raise ValueError(f"jacobi requires a square matrix, got {A.shape}.")
    shifted = csr_diagonal(A) + float(shift)
    if not bool(torch.isfinite(shifted).all()):
        raise ValueError("shifted diagonal must contain only finite values.")
    if zero_atol < 0.0:
        raise ValueError("zero_atol must be non-negative.")
    near_zero = shifted.abs() <= zero_atol
    if check and not bool((shifted > zero_atol).all()):
        raise ValueError("Jacobi shifted diagonal must be strictly positive when check=True.")
    if bool(near_zero.any()):
        if zero_policy == "raise":
            raise ValueError("Jacobi shifted diagonal contains zero or near-zero entries.")
        shifted = torch.where(near_zero, torch.ones_like(shifted), shifted)
    return JacobiPreconditioner(float(omega) / shifted, A.shape, omega=float(omega),
                                shift=float(shift))


def aspreconditioner(M, A=None):
    """Normalise ``M`` for the native solvers: preconditioner objects pass
    through; a rank-1 tensor is taken as an inverse diagonal."""
    if isinstance(M, (IdentityPreconditioner, DiagonalPreconditioner)):
        return M
    if isinstance(M, torch.Tensor) and M.ndim == 1:
        return diagonal(M, inverse=True)
    if isinstance(M, CSRArray):
        # reference: mlx_sparse/linalg/preconditioners.py:1585-1590
        raise TypeError("sparse matrices are not inverse-apply preconditioners; use "
                        "preconditioners.jacobi(A) or preconditioners.diagonal(...).")
    raise TypeError(
        "cg currently supports only identity, diagonal and Jacobi native-backed preconditioners.")
