"""CSR container (reference: mlx_sparse/_csr.py:33-129 ``CSRArray``,
:502-552 ``__matmul__``, :627-730 ``csr_array``).

``CSRArray`` is a frozen dataclass over three torch tensors.  It caches, per
device, copies of its buffers, the GPU plan bound to them and its transpose
(built on first use, released with the array).  The reference's arrays are
immutable; torch tensors are not, so every cache entry records what it was
built from - each tensor's storage address and version counter, which every
in-place operation bumps - and is brought up to date on its next use:

- new values (``A.data`` updated in place, e.g. by an optimizer step): device
  copies are copied again, the plan's reordered copy of the values is
  rewritten through the layout it holds (``CSRPlan.refresh``, one pass over
  the values), and a cached transpose gets its values regathered through
  the stored position of every entry (computed once), as a new array that
  takes over the old one's plan;
- new ``indices`` or ``indptr``: plans and transposes are built again.

Writes that torch does not count (through ``.data``, DLPack or raw
pointers) are not seen.
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


def _stamp(t: torch.Tensor) -> tuple[int, int]:
    """Storage address and version counter of a tensor: what a cache entry
    built from it must still match.  Inference tensors keep no version
    counter; they count as unchanged while their storage is."""
    try:
        return (t.data_ptr(), t._version)
    except RuntimeError:
        return (t.data_ptr(), -1)


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
    def _stamps(self) -> tuple:
        return (_stamp(self.data), _stamp(self.indices), _stamp(self.indptr))

    def buffers(self, device) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """``(data, indices, indptr)`` contiguous on ``device`` (cached; a
        tensor already contiguous on ``device`` is used as it is, a copy is
        made again when its source changed)."""
        device = torch.device(device)
        if device.type == "cuda" and device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        key = ("buffers", str(device))
        now = self._stamps()
        hit = self._cache.get(key)
        if hit is not None and hit[0] == now:
            return hit[1]
        old_stamps, old = hit if hit is not None else ((None,) * 3, (None,) * 3)
        bufs = tuple(
            o if o is not None and was == cur else t.to(device).contiguous()
            for t, o, was, cur in zip((self.data, self.indices, self.indptr), old, old_stamps, now))
        self._cache[key] = (now, bufs)
        return bufs

    def plan(self, device=None):
        """The GPU plan for ``device``, bound to :meth:`buffers` (None on the
        CPU, or when the ``gpu_plan`` runtime option is off).  Built once;
        refreshed when the values changed, rebuilt when the structure did."""
        from mlx_sparse import runtime

        device = torch.device(device) if device is not None else self.device
        if device.type != "cuda" or not runtime.get(runtime.RuntimeOption.GPU_PLAN):
            return None
        data, indices, indptr = self.buffers(device)
        key = ("plan", str(indptr.device))
        now = self._stamps()
        hit = self._cache.get(key)
        if hit is not None:
            built, plan = hit
            if built[1:] == now[1:]:
                if built[0] != now[0]:
                    plan.refresh(data)
                    self._cache[key] = (now, plan)
                return plan
        from mlx_sparse import _native

        # bound to these buffers: may hold a reordered copy of the values
        plan = _native.csr_plan(indptr, self.shape[0], self.nnz, data=data, indices=indices,
                                n_cols=self.shape[1],
                                slice_mode=int(runtime.get(runtime.RuntimeOption.GPU_SLICE)))
        self._cache[key] = (now, plan)
        return plan

    def _with_values(self, data: torch.Tensor) -> "CSRArray":
        """The same structure with other values, taking over this array's
        GPU plans (each is rebound to ``data`` on its next use, as after an
        in-place update); this array builds new ones if it is used again."""
        out = CSRArray(data=data, indices=self.indices, indptr=self.indptr, shape=self.shape,
                       sorted_indices=self.sorted_indices,
                       has_canonical_format=self.has_canonical_format)
        for key in [k for k in self._cache if k[0] == "plan"]:
            built, plan = self._cache.pop(key)
            out._cache[key] = (((None, None),) + tuple(built[1:]), plan)
        return out

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
    def _transpose_on(self, device, conjugate: bool = False) -> "CSRArray":
        """CSR of the transpose (of the conjugate transpose with
        ``conjugate``), computed on ``device``.  Cached while this array is
        unchanged; after new values, the cached transpose's values are
        regathered on the GPU in two streaming passes through a layout
        computed, on the first such update, from the stored position of each
        of its entries (8 bytes per value), as a new array."""
        from mlx_sparse import _native

        device = torch.device(device)
        data, indices, indptr = self.buffers(device)
        key = ("H" if conjugate else "T", str(data.device))
        now = self._stamps()
        hit = self._cache.get(key)
        if hit is not None:
            built, T, layout = hit
            if built == now:
                return T
            if built[1:] == now[1:] and data.device.type == "cuda":
                if layout is None:
                    pos = _native.csr_transpose_positions(indices, indptr, self.shape)[0]
                    layout = _native.csr_transpose_layout(pos, T.data)
                    del pos
                t_data = torch.empty_like(T.data)
                scratch = torch.empty_like(T.data)
                _native.csr_transpose_values_layout(data.detach(), layout, conjugate, scratch, t_data)
                T = T._with_values(t_data)
                self._cache[key] = (now, T, layout)
                return T
        src = data.detach()
        if conjugate:
            src = src.conj().resolve_conj()
        t_data, t_indices, t_indptr = _native.csr_transpose(src, indices, indptr, self.shape)
        T = CSRArray(
            data=t_data,
            indices=t_indices,
            indptr=t_indptr,
            shape=(self.shape[1], self.shape[0]),
            sorted_indices=True,
            has_canonical_format=self.has_canonical_format,
        )
        self._cache[key] = (now, T, None)
        return T

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
        """Hermitian (conjugate) transpose, ``conj().T``: for real values the
        transpose itself; both are cached like :meth:`transpose`."""
        from mlx_sparse._device import default_torch_device

        return self._transpose_on(default_torch_device(), conjugate=self.data.is_complex())

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
