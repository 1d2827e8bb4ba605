"""Public operator wrappers for the CSR sparse x dense path (reference:
mlx_sparse/_ops.py:780-818 ``csr_matvec``, :972-1000 rank-2/batched helpers,
:1118-1167 ``csr_matmul``).

Operations run on the selected device (``use_cpu``/``use_gpu``); operands
are moved there first.  GPU SpMV uses the matrix's cached row-block plan.
Unlike MLX the result is not lazy: the kernel is enqueued on torch's current
stream and the returned tensor is ordered after it, which composes with any
torch operation on that stream.
"""

from __future__ import annotations

import math

import torch

import mlx_sparse._native as _native
from mlx_sparse._csr import CSRArray
from mlx_sparse._device import default_torch_device
from mlx_sparse._validation import (
    ensure_array,
    validate_csr_matmul_inputs,
    validate_csr_matvec_inputs,
)


def _prod(shape) -> int:
    return int(math.prod(int(d) for d in shape))


def _tracked(*tensors: torch.Tensor) -> bool:
    """True when the product must carry derivatives: reverse mode (grad
    enabled and an operand requires grad), forward mode (a dual level is
    open) or a torch.func transform (vmap, grad, jvp) is active."""
    if torch._C._are_functorch_transforms_active():
        return True
    if torch.is_grad_enabled() and any(t.requires_grad for t in tensors):
        return True
    from torch.autograd import forward_ad

    return forward_ad._current_level >= 0


def csr_matvec(a: CSRArray, x) -> torch.Tensor:
    """Multiply a CSR sparse matrix by a dense vector: ``y = A @ x``.

    Args:
        a: The sparse matrix, shape ``(n_rows, n_cols)``.
        x: Dense vector, shape ``(n_cols,)``, same dtype as ``a.data``.

    Returns:
        Dense vector of shape ``(n_rows,)`` with the dtype of ``a.data``.

    Raises:
        TypeError: ``a`` is not a CSRArray, or the dtypes of ``a.data`` and
            ``x`` differ or are unsupported.
        ValueError: shape constraints are violated.
    """
    if not isinstance(a, CSRArray):
        raise TypeError(f"csr_matvec expects CSRArray, got {type(a).__name__}.")
    device = default_torch_device()
    x = ensure_array(x, device=device)
    validate_csr_matvec_inputs(a.data, a.indices, a.indptr, x, a.shape)
    if _tracked(a.data, x):
        from mlx_sparse._autograd import CSRMatVec

        return CSRMatVec.apply(a.data.to(x.device), x, a, True)
    data, indices, indptr = a.buffers(device)
    return _native.csr_matvec(data, indices, indptr, x, a.shape, plan=a.plan(device))


def _csr_matmul_rank2(a: CSRArray, rhs: torch.Tensor) -> torch.Tensor:
    validate_csr_matmul_inputs(a.data, a.indices, a.indptr, rhs, a.shape)
    if _tracked(a.data, rhs):
        from mlx_sparse._autograd import CSRMatMul

        return CSRMatMul.apply(a.data.to(rhs.device), rhs, a, True)
    data, indices, indptr = a.buffers(rhs.device)
    # the cached bound plan carries the column windows of the row tiles
    return _native.csr_matmul(data, indices, indptr, rhs, a.shape, plan=a.plan(rhs.device))


def _csr_matmul_batched(a: CSRArray, rhs: torch.Tensor) -> torch.Tensor:
    """``out[b] = A @ rhs[b]`` over the flattened leading dimensions, through
    the native batched SpMM (reference: mlx_sparse/_ops.py:986-1000)."""
    if a.data.dtype != rhs.dtype:
        raise TypeError(
            "csr_matmul requires sparse data and RHS to have the same dtype, "
            f"got {a.data.dtype} and {rhs.dtype}."
        )
    batch_shape = tuple(int(d) for d in rhs.shape[:-2])
    k = int(rhs.shape[-1])
    if _tracked(a.data, rhs):
        # one rank-2 product over the batch laid side by side: every output
        # is still summed from zero in stored order, so the values equal the
        # batched kernel's, and the rank-2 rules give the derivatives
        from mlx_sparse._autograd import CSRMatMul

        B = _prod(batch_shape)
        wide = rhs.reshape(B, a.shape[1], k).permute(1, 0, 2).reshape(a.shape[1], B * k)
        out = CSRMatMul.apply(a.data.to(rhs.device), wide, a, True)
        out = out.reshape(a.shape[0], B, k).permute(1, 0, 2)
        return out.reshape(*batch_shape, a.shape[0], k)
    flat = rhs.reshape(_prod(batch_shape), a.shape[1], k)
    data, indices, indptr = a.buffers(rhs.device)
    out = _native.csr_batched_matmul(data, indices, indptr, flat, a.shape)
    return out.reshape(*batch_shape, a.shape[0], k)


def csr_matmul(a: CSRArray, rhs) -> torch.Tensor:
    """Multiply a CSR sparse matrix by a dense matrix: ``Y = A @ B``.

    ``rhs`` is ``(n_cols, k)`` or batched ``(..., n_cols, k)``.

    Raises:
        TypeError: ``a`` is not a CSRArray or dtypes are violated.
        ValueError: shape constraints are violated.
    """
    if not isinstance(a, CSRArray):
        raise TypeError(f"csr_matmul expects CSRArray, got {type(a).__name__}.")
    rhs = ensure_array(rhs, device=default_torch_device())
    if rhs.ndim == 2:
        return _csr_matmul_rank2(a, rhs)
    if rhs.ndim < 2:
        raise ValueError(f"csr_matmul expects rank-2 or higher RHS, got {tuple(rhs.shape)}.")
    if rhs.shape[-2] != a.shape[1]:
        raise ValueError(
            f"csr_matmul RHS has sparse dimension {rhs.shape[-2]}, "
            f"but sparse n_cols={a.shape[1]}."
        )
    return _csr_matmul_batched(a, rhs)


def csr_batched_matvec(a: CSRArray, rhs) -> torch.Tensor:
    """Multiply a CSR sparse matrix by a batch of dense vectors: ``Y[b] = A @
    X[b]`` for ``rhs`` of shape ``(..., n_cols)``; returns ``(..., n_rows)``
    (reference: mlx_sparse/_ops.py:821-855).  Each output is summed from zero
    in stored order, as the reference's batched kernels sum it.

    Raises:
        TypeError: ``a`` is not a CSRArray or the dtypes differ.
        ValueError: ``rhs`` has rank < 2 or the wrong vector length.
    """
    if not isinstance(a, CSRArray):
        raise TypeError(f"csr_batched_matvec expects CSRArray, got {type(a).__name__}.")
    rhs = ensure_array(rhs, device=default_torch_device())
    if rhs.ndim < 2:
        raise ValueError(
            f"csr_batched_matvec expects rank-2 or higher RHS, got {tuple(rhs.shape)}."
        )
    if rhs.shape[-1] != a.shape[1]:
        raise ValueError(
            f"csr_batched_matvec RHS has vector dimension {rhs.shape[-1]}, "
            f"but sparse n_cols={a.shape[1]}."
        )
    if a.data.dtype != rhs.dtype:
        raise TypeError(
            "csr_batched_matvec requires sparse data and RHS to have the same dtype, "
            f"got {a.data.dtype} and {rhs.dtype}."
        )
    batch_shape = tuple(int(d) for d in rhs.shape[:-1])
    flat = rhs.reshape(_prod(batch_shape), a.shape[1])
    if _tracked(a.data, rhs):
        # the batch as the columns of one rank-2 product (zero-start stored
        # order, as the batched kernel sums)
        from mlx_sparse._autograd import CSRMatMul

        out = CSRMatMul.apply(a.data.to(rhs.device), flat.transpose(0, 1), a, True)
        return out.transpose(0, 1).reshape(*batch_shape, a.shape[0])
    data, indices, indptr = a.buffers(rhs.device)
    out = _native.csr_batched_matvec(data, indices, indptr, flat, a.shape)
    return out.reshape(*batch_shape, a.shape[0])


def csr_batched_matmul(a: CSRArray, rhs) -> torch.Tensor:
    """Multiply a CSR sparse matrix by a batch of dense matrices: ``rhs`` of
    shape ``(..., n_cols, k)`` gives ``(..., n_rows, k)`` (reference:
    mlx_sparse/_ops.py:1097-1115).  For rank-2 ``rhs`` use ``csr_matmul``."""
    if not isinstance(a, CSRArray):
        raise TypeError(f"csr_batched_matmul expects CSRArray, got {type(a).__name__}.")
    rhs = ensure_array(rhs, device=default_torch_device())
    if rhs.ndim < 3:
        raise ValueError(
            f"csr_batched_matmul expects rank-3 or higher RHS, got {tuple(rhs.shape)}."
        )
    if rhs.shape[-2] != a.shape[1]:
        raise ValueError(
            f"csr_batched_matmul RHS has sparse dimension {rhs.shape[-2]}, "
            f"but sparse n_cols={a.shape[1]}."
        )
    return _csr_matmul_batched(a, rhs)


def csr_matvec_transpose(a: CSRArray, x) -> torch.Tensor:
    """``A^T x`` without materialising the transpose (no conjugation), for
    ``x`` of shape ``(n_rows,)`` (reference: mlx_sparse/_native.py:260-270).
    GPU: atomic scatter over A's rows; CPU: per-range partial outputs added in
    range order, as in the reference.  For ``A.T @ x`` through the
    materialised transpose use ``a.T @ x``."""
    if not isinstance(a, CSRArray):
        raise TypeError(f"csr_matvec_transpose expects CSRArray, got {type(a).__name__}.")
    device = default_torch_device()
    x = ensure_array(x, device=device)
    if x.ndim != 1 or x.shape[0] != a.shape[0]:
        raise ValueError(
            f"csr_matvec_transpose expects x of shape ({a.shape[0]},), got {tuple(x.shape)}.")
    if x.dtype != a.data.dtype:
        raise TypeError("csr_matvec_transpose requires data and x to have the same dtype.")
    data, indices, indptr = a.buffers(device)
    return _native.csr_matvec_transpose(data, indices, indptr, x, a.shape)


def csr_matmul_transpose(a: CSRArray, rhs) -> torch.Tensor:
    """``A^T X`` without materialising the transpose, for ``rhs`` of shape
    ``(n_rows, k)`` (reference: mlx_sparse/_native.py:367-377)."""
    if not isinstance(a, CSRArray):
        raise TypeError(f"csr_matmul_transpose expects CSRArray, got {type(a).__name__}.")
    device = default_torch_device()
    rhs = ensure_array(rhs, device=device)
    if rhs.ndim != 2 or rhs.shape[0] != a.shape[0]:
        raise ValueError(
            f"csr_matmul_transpose expects rhs of shape ({a.shape[0]}, k), "
            f"got {tuple(rhs.shape)}.")
    if rhs.dtype != a.data.dtype:
        raise TypeError("csr_matmul_transpose requires data and rhs to have the same dtype.")
    data, indices, indptr = a.buffers(device)
    return _native.csr_matmul_transpose(data, indices, indptr, rhs, a.shape)
