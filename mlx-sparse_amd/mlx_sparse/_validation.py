"""Python-side validation (reference: mlx_sparse/_validation.py:43-339).

Same checks, order and texts as the reference for the CSR sparse x dense
path; ``TypeError`` for dtypes and ``ValueError`` for shapes, raised before
any native call and without reading array values (except ``validate="full"``).
"""

from __future__ import annotations

from collections.abc import Sequence

import numpy as np
import torch

from mlx_sparse._typing import INDEX_DTYPES, VALUE_DTYPES, Shape2D, ValidationMode


def normalize_shape(shape: Sequence[int]) -> Shape2D:
    if len(shape) != 2:
        raise ValueError(f"sparse arrays must be rank-2, got shape={tuple(shape)!r}.")
    n_rows, n_cols = int(shape[0]), int(shape[1])
    if n_rows < 0 or n_cols < 0:
        raise ValueError(f"sparse dimensions must be non-negative, got {shape!r}.")
    return n_rows, n_cols


def normalize_validation_mode(validate: ValidationMode) -> str:
    if validate is True:
        return "full"
    if validate is False:
        return "none"
    if validate not in {"metadata", "full"}:
        raise ValueError(
            "validate must be one of False, True, 'metadata', or 'full', "
            f"got {validate!r}."
        )
    return validate


def ensure_array(value, *, dtype=None, device=None) -> torch.Tensor:
    """Convert to a tensor on ``device`` (the default device when None)."""
    from mlx_sparse._device import default_torch_device

    target = default_torch_device() if device is None else torch.device(device)
    if isinstance(value, torch.Tensor):
        t = value
    elif isinstance(value, np.ndarray):
        t = torch.from_numpy(np.ascontiguousarray(value))
    else:
        t = torch.as_tensor(value)
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    if t.device != target:
        t = t.to(target)
    return t


def _shape(array) -> tuple:
    return tuple(int(d) for d in array.shape)


def check_rank1(name: str, array: torch.Tensor) -> None:
    if array.ndim != 1:
        raise ValueError(f"{name} must be rank-1, got shape={_shape(array)}.")


def _names(dtypes) -> str:
    return ", ".join(str(dt).split(".")[-1] for dt in dtypes)


def check_index_dtype(name: str, array: torch.Tensor) -> None:
    if array.dtype not in INDEX_DTYPES:
        raise TypeError(f"{name} dtype must be one of {_names(INDEX_DTYPES)}, got {array.dtype}.")


def check_value_dtype(name: str, array: torch.Tensor) -> None:
    if array.dtype not in VALUE_DTYPES:
        raise TypeError(f"{name} dtype must be one of {_names(VALUE_DTYPES)}, got {array.dtype}.")


def validate_csr_metadata(data, indices, indptr, shape: Shape2D) -> None:
    check_rank1("CSRArray.data", data)
    check_rank1("CSRArray.indices", indices)
    check_rank1("CSRArray.indptr", indptr)
    check_value_dtype("CSRArray.data", data)
    check_index_dtype("CSRArray.indices", indices)
    check_index_dtype("CSRArray.indptr", indptr)
    if indices.dtype != indptr.dtype:
        raise TypeError(
            "CSRArray indices and indptr must have the same dtype, "
            f"got {indices.dtype} and {indptr.dtype}."
        )
    if data.shape[0] != indices.shape[0]:
        raise ValueError(
            "CSRArray data and indices must have the same length, "
            f"got {data.shape[0]} and {indices.shape[0]}."
        )
    expected_indptr = shape[0] + 1
    if indptr.shape[0] != expected_indptr:
        raise ValueError(
            "CSRArray indptr must have shape (n_rows + 1,), "
            f"got {_shape(indptr)} for n_rows={shape[0]}."
        )


def validate_csr_values(indices, indptr, shape: Shape2D, nnz: int) -> None:
    indices_np = indices.detach().cpu().numpy()
    indptr_np = indptr.detach().cpu().numpy()
    if indptr_np[0] != 0:
        raise ValueError(f"CSRArray indptr[0] must be 0, got {indptr_np[0]}.")
    if indptr_np[-1] != nnz:
        raise ValueError(f"CSRArray indptr[-1] must equal nnz={nnz}, got {indptr_np[-1]}.")
    if (indptr_np[1:] < indptr_np[:-1]).any():
        raise ValueError("CSRArray indptr must be monotonically nondecreasing.")
    if indices_np.size:
        min_index = int(indices_np.min())
        max_index = int(indices_np.max())
        if min_index < 0 or max_index >= shape[1]:
            raise ValueError(
                "CSRArray indices must be in bounds for n_cols="
                f"{shape[1]}, got min={min_index}, max={max_index}."
            )


def validate_csr_matvec_inputs(data, indices, indptr, x, shape: Shape2D) -> None:
    validate_csr_metadata(data, indices, indptr, shape)
    if x.ndim != 1:
        raise ValueError(f"csr_matvec expects a rank-1 RHS, got shape={_shape(x)}.")
    if x.shape[0] != shape[1]:
        raise ValueError(
            f"csr_matvec RHS has length {x.shape[0]}, but sparse n_cols={shape[1]}."
        )
    check_value_dtype("csr_matvec data", data)
    check_value_dtype("csr_matvec RHS", x)
    if data.dtype != x.dtype:
        raise TypeError(
            "csr_matvec requires sparse data and RHS to have the same dtype, "
            f"got {data.dtype} and {x.dtype}."
        )


def validate_csr_matmul_inputs(data, indices, indptr, rhs, shape: Shape2D) -> None:
    validate_csr_metadata(data, indices, indptr, shape)
    if rhs.ndim != 2:
        raise ValueError(f"csr_matmul expects a rank-2 RHS, got shape={_shape(rhs)}.")
    if rhs.shape[0] != shape[1]:
        raise ValueError(
            f"csr_matmul RHS has leading dimension {rhs.shape[0]}, "
            f"but sparse n_cols={shape[1]}."
        )
    check_value_dtype("csr_matmul data", data)
    check_value_dtype("csr_matmul RHS", rhs)
    if data.dtype != rhs.dtype:
        raise TypeError(
            "csr_matmul requires sparse data and RHS to have the same dtype, "
            f"got {data.dtype} and {rhs.dtype}."
        )
