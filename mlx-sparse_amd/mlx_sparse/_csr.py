"""CSR container (reference: mlx_sparse/_csr.py:33-129 ``CSRArray``,
:502-552 ``__matmul__``, :627-730 ``csr_array``).

``CSRArray`` is an immutable dataclass over three torch tensors.  Because it
is immutable it can cache, per device, copies of its buffers and the GPU
row-block plan built from ``indptr`` (built on first use, released with the
array).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from mlx_sparse._typing import Shape2D, ValidationMode
from mlx_sparse._validation import (
    ensure_array,
    normalize_shape,
    normalize_validation_mode,
    validate_csr_metadata,
    validate_csr_values,
)


@dataclass(frozen=True, slots=True)
class CSRArray:
    """A 2D sparse matrix in Compressed Sparse Row (CSR) format.

    - **data**: non-zero values, shape ``(nnz,)``, float32, float16,
      bfloat16 or complex64.
    - **indices**: column index of each stored value, shape ``(nnz,)``.
    - **indptr**: row pointers, shape ``(n_rows + 1,)``, same integer dtype as
      ``indices`` (int32 or int64).

    Row ``i`` spans ``data[indptr[i]:indptr[i+1]]``.  ``A @ x`` runs CSR SpMV,
    ``A @ X`` CSR SpMM, on the device selected with ``use_cpu``/``use_gpu``.
    """

    data: torch.Tensor
    indices: torch.Tensor
    indptr: torch.Tensor
    shape: Shape2D
    sorted_indices: bool = False
    has_canonical_format: bool = False
    _cache: dict = field(default_factory=dict, compare=False, repr=False, hash=False)

    def __post_init__(self) -> None:
        object.__setattr__(self, "shape", normalize_shape(self.shape))

    @property
    def nnz(self) -> int:
        """Number of stored values (including duplicates)."""
        return int(self.data.shape[0])

    @property
    def dtype(self):
        return self.data.dtype

    @property
    def index_dtype(self):
        return self.indices.dtype

    @property
    def ndim(self) -> int:
        return 2

    @property
    def device(self) -> torch.device:
        return self.data.device

    def __repr__(self) -> str:
        return (
            "CSRArray("
            f"shape={self.shape}, nnz={self.nnz}, dtype={self.dtype}, "
            f"index_dtype={self.index_dtype}, "
            f"sorted_indices={self.sorted_indices}, "
            f"has_canonical_format={self.has_canonical_format})"
        )

    # -- device copies and plans -----------------------------------------
    def buffers(self, device) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """``(data, indices, indptr)`` contiguous on ``device`` (cached)."""
        device = torch.device(device)
        if device.type == "cuda" and device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        key = ("buffers", str(device))
        hit = self._cache.get(key)
        if hit is None:
            hit = tuple(t.to(device).contiguous() for t in (self.data, self.indices, self.indptr))
            self._cache[key] = hit
        return hit

    def plan(self, device=None):
        """The GPU row-block plan for ``device`` (None on the CPU, or when the
        ``gpu_plan`` runtime option is off).  Built once, then cached."""
        from mlx_sparse import runtime

        device = torch.device(device) if device is not None else self.device
        if device.type != "cuda" or not runtime.get(runtime.RuntimeOption.GPU_PLAN):
            return None
        data, indices, indptr = self.buffers(device)
        key = ("plan", str(indptr.device))
        hit = self._cache.get(key)
        if hit is None:
            from mlx_sparse import _native

            # bound to this immutable matrix: may hold a column-sliced copy
            hit = _native.csr_plan(indptr, self.shape[0], self.nnz, data=data, indices=indices,
                                   n_cols=self.shape[1],
                                   slice_mode=int(runtime.get(runtime.RuntimeOption.GPU_SLICE)))
            self._cache[key] = hit
        return hit

    # -- operators ---------------------------------------------------------
    def __matmul__(self, rhs):
        """``A @ rhs``: rank-1 dense ``rhs`` -> :func:`csr_matvec`, rank >= 2
        -> :func:`csr_matmul` (batched over leading dimensions)."""
        if isinstance(rhs, CSRArray):
            raise NotImplementedError("sparse x sparse products are outside this build.")
        if not isinstance(rhs, torch.Tensor):
            rhs = ensure_array(rhs)
        if rhs.ndim == 1:
            from mlx_sparse._ops import csr_matvec

            return csr_matvec(self, rhs)
        if rhs.ndim >= 2:
            from mlx_sparse._ops import csr_matmul

            return csr_matmul(self, rhs)
        raise ValueError(f"CSR matmul expects rank-1 or higher RHS, got {tuple(rhs.shape)}.")

    # -- transpose and conjugate -------------------------------------------
    def _transpose_on(self, device) -> "CSRArray":
        """CSR of the transpose, computed on ``device`` (cached: the array is
        immutable)."""
        device = torch.device(device)
        data, indices, indptr = self.buffers(device)
        key = ("T", str(data.device))
        hit = self._cache.get(key)
        if hit is None:
            from mlx_sparse import _native

            t_data, t_indices, t_indptr = _native.csr_transpose(data.detach(), indices, indptr,
                                                                self.shape)
            hit = CSRArray(
                data=t_data,
                indices=t_indices,
                indptr=t_indptr,
                shape=(self.shape[1], self.shape[0]),
                sorted_indices=True,
                has_canonical_format=self.has_canonical_format,
            )
            self._cache[key] = hit
        return hit

    def transpose(self) -> "CSRArray":
        """Transpose, returning a ``CSRArray`` of shape ``(n_cols, n_rows)``
        with ``sorted_indices=True`` (each row lists its values by increasing
        column, duplicates in stored order) and the source's
        ``has_canonical_format`` (reference: mlx_sparse/_csr.py:252-275).
        Computed on the selected device; the values are not differentiable
        through it, as in the reference."""
        from mlx_sparse._device import default_torch_device

        return self._transpose_on(default_torch_device())

    @property
    def T(self) -> "CSRArray":
        """Transposed matrix. Alias for :meth:`transpose`."""
        return self.transpose()

    def conj(self) -> "CSRArray":
        """Complex-conjugate the stored values; the structure is shared
        (reference: mlx_sparse/_csr.py:362-379)."""
        data = self.data.conj().resolve_conj() if self.data.is_complex() else self.data
        return CSRArray(
            data=data,
            indices=self.indices,
            indptr=self.indptr,
            shape=self.shape,
            sorted_indices=self.sorted_indices,
            has_canonical_format=self.has_canonical_format,
        )

    def conjugate(self) -> "CSRArray":
        """Alias for :meth:`conj`."""
        return self.conj()

    @property
    def H(self) -> "CSRArray":
        """Hermitian (conjugate) transpose, ``conj().T``."""
        return self.conj().transpose()

    def todense(self) -> torch.Tensor:
        """Dense copy (duplicates summed), on the buffers' device."""
        n_rows, n_cols = self.shape
        rows = torch.repeat_interleave(
            torch.arange(n_rows, device=self.indptr.device),
            (self.indptr[1:] - self.indptr[:-1]).to(torch.int64),
        )
        out = torch.zeros(n_rows * n_cols, dtype=self.dtype, device=self.data.device)
        flat = rows.to(torch.int64) * n_cols + self.indices.to(torch.int64)
        out.index_add_(0, flat, self.data)
        return out.reshape(n_rows, n_cols)


def csr_array(
    arg,
    shape,
    *,
    validate: ValidationMode = "metadata",
    sorted_indices: bool = False,
    canonical: bool | None = None,
) -> CSRArray:
    """Construct a :class:`CSRArray` from ``(data, indices, indptr)``.

    Buffers (torch tensors, numpy arrays or sequences) are placed on the
    selected device.  ``validate="metadata"`` checks ranks, lengths and
    dtypes without reading values; ``"full"``/``True`` also checks indptr
    monotonicity and column bounds (host sync); ``False`` skips checks.
    """
    mode = normalize_validation_mode(validate)
    shape = normalize_shape(shape)
    if isinstance(arg, CSRArray):
        if arg.shape != shape:
            raise ValueError(f"CSRArray shape mismatch: got {arg.shape}, expected {shape}.")
        return arg
    try:
        data, indices, indptr = arg
    except Exception as exc:
        raise TypeError(
            "csr_array expects (data, indices, indptr) or a CSRArray instance."
        ) from exc
    data = ensure_array(data)
    indices = ensure_array(indices)
    indptr = ensure_array(indptr)
    if mode != "none":
        validate_csr_metadata(data, indices, indptr, shape)
    if mode == "full":
        validate_csr_values(indices, indptr, shape, data.shape[0])
    has_canonical_format = bool(canonical) if canonical is not None else False
    if has_canonical_format:
        sorted_indices = True
    return CSRArray(
        data=data,
        indices=indices,
        indptr=indptr,
        shape=shape,
        sorted_indices=sorted_indices,
        has_canonical_format=has_canonical_format,
    )
