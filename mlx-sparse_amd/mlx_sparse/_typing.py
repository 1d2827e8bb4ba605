"""Dtype sets and shared aliases (reference: mlx_sparse/_typing.py:15-73).

Arrays are ``torch.Tensor``: MLX has no ROCm backend, so PyTorch-ROCm holds
device memory and streams.  The supported dtypes are the reference's.
"""

from __future__ import annotations

from typing import Callable, Literal, TypeAlias

import torch

Shape2D: TypeAlias = tuple[int, int]
ValidationMode: TypeAlias = bool | Literal["metadata", "full"]

INDEX_DTYPES = (torch.int32, torch.int64)
VALUE_DTYPES = (torch.float32, torch.float16, torch.bfloat16, torch.complex64)

Matvec = Callable[[torch.Tensor], torch.Tensor]
Matmat = Callable[[torch.Tensor], torch.Tensor]


def is_index_dtype(dtype) -> bool:
    return dtype in INDEX_DTYPES


def is_supported_value_dtype(dtype) -> bool:
    return dtype in VALUE_DTYPES


def is_available() -> bool:
    """Return ``True`` if the native extension (``mlx_sparse._ext``) loads.

    Unlike the reference there is no NumPy fallback: without the extension
    every operation raises.
    """
    from mlx_sparse._ext_loader import extension_available

    return extension_available()
