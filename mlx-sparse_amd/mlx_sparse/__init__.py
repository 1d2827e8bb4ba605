"""mlx_sparse on MI355X: the CSR sparse x dense path of mlx-sparse
(``csr_array``, ``A @ x``, ``A @ X``), on PyTorch-ROCm tensors and
hand-written gfx950 HIP kernels behind the C ABI in ``include/msx_sparse.h``.
"""

from __future__ import annotations

from mlx_sparse import linalg, runtime
from mlx_sparse._csr import CSRArray, csr_array
from mlx_sparse._device import default_torch_device, use_cpu, use_device, use_gpu
from mlx_sparse._io import from_scipy, mminfo, mmread
from mlx_sparse._ops import (
    csr_batched_matmul,
    csr_batched_matvec,
    csr_matmul,
    csr_matmul_transpose,
    csr_matvec,
    csr_matvec_transpose,
)
from mlx_sparse._typing import INDEX_DTYPES, VALUE_DTYPES, is_available


def capabilities() -> dict:
    """Compile-time facts of the native module (reference
    mlx_sparse/_capabilities.py:279-322 reports the same keys)."""
    from mlx_sparse._ext_loader import extension

    return dict(extension()._compiled_capabilities())


__all__ = [
    "CSRArray",
    "INDEX_DTYPES",
    "VALUE_DTYPES",
    "capabilities",
    "csr_array",
    "csr_batched_matmul",
    "csr_batched_matvec",
    "csr_matmul",
    "csr_matmul_transpose",
    "csr_matvec",
    "csr_matvec_transpose",
    "default_torch_device",
    "from_scipy",
    "is_available",
    "linalg",
    "mminfo",
    "mmread",
    "runtime",
    "use_cpu",
    "use_device",
    "use_gpu",
]
