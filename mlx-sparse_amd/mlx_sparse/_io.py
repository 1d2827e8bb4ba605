"""Input formats: Matrix Market files and SciPy sparse matrices into
``CSRArray`` (reference: ``from_scipy``, mlx_sparse/_construct.py:854-975;
its tests read the SuiteSparse fixtures with scipy.io.mmread,
tests/test_suitesparse_collection.py:36-47).

``mmread`` parses in native code (the library's Matrix Market reader:
multithreaded, symmetric kinds expanded, canonical CSR out) and places the
buffers on the selected device.
"""

from __future__ import annotations

import os

import numpy as np
import torch

from mlx_sparse._csr import CSRArray
from mlx_sparse._device import default_torch_device
from mlx_sparse._ext_loader import extension
from mlx_sparse._typing import INDEX_DTYPES, VALUE_DTYPES


def _value_dtype(dtype, field: str | None = None) -> torch.dtype:
    if dtype is None:
        return torch.complex64 if field == "complex" else torch.float32
    if dtype not in VALUE_DTYPES:
        raise TypeError(f"dtype must be one of float32, float16, bfloat16, complex64, got {dtype}.")
    return dtype


def _index_dtype(index_dtype) -> torch.dtype:
    if index_dtype not in INDEX_DTYPES:
        raise TypeError(f"index_dtype must be int32 or int64, got {index_dtype}.")
    return index_dtype


def mminfo(source) -> tuple[int, int, int, str, str, str]:
    """``(rows, cols, entries, format, field, symmetry)`` of a Matrix Market
    file, as ``scipy.io.mminfo`` reports them."""
    d = extension().mm_info(os.fspath(source))
    return d["rows"], d["cols"], d["entries"], d["format"], d["field"], d["symmetry"]


def mmread(source, *, dtype=None, index_dtype=torch.int32, n_threads: int = 0):
    """Read a Matrix Market file.  Coordinate files give a canonical
    :class:`CSRArray` (symmetric kinds expanded, rows sorted, duplicates
    summed); array files give a dense tensor.  ``dtype`` defaults to float32
    (complex64 for complex files); values are rounded once from the file's
    decimal text.  Buffers land on the selected device."""
    path = os.fspath(source)
    ext = extension()
    info = ext.mm_info(path)
    vdt = _value_dtype(dtype, info["field"])
    if info["field"] == "complex" and vdt != torch.complex64:
        raise TypeError("a complex Matrix Market file needs dtype complex64.")
    device = default_torch_device()
    if info["format"] == "array":
        return ext.mm_read_dense(path, vdt, n_threads).to(device)
    data, indices, indptr, shape = ext.mm_read_csr(path, vdt, _index_dtype(index_dtype), n_threads)
    return CSRArray(data=data.to(device), indices=indices.to(device), indptr=indptr.to(device),
                    shape=tuple(shape), sorted_indices=True, has_canonical_format=True)


def _numpy_value_dtype(values: np.ndarray, dtype) -> torch.dtype:
    if dtype is not None:
        return _value_dtype(dtype)
    if np.iscomplexobj(values):
        return torch.complex64
    if values.dtype == np.float16:
        return torch.float16
    return torch.float32


def from_scipy(matrix, *, format: str = "csr", dtype=None, index_dtype=torch.int32,
               canonical: bool = True) -> CSRArray:
    """Convert a SciPy sparse matrix or array to a :class:`CSRArray`.

    Values keep float32 / float16 / complex64; other real dtypes (SciPy's
    float64 default included) become float32 unless ``dtype`` says
    otherwise.  ``canonical`` sums duplicates and sorts indices first.  Only
    ``format="csr"`` exists in this build (the path's format)."""
    try:
        import scipy.sparse as sp
    except ImportError as exc:  # pragma: no cover
        raise TypeError("from_scipy requires scipy to be installed.") from exc
    if not sp.issparse(matrix):
        raise TypeError(
            f"from_scipy expects a scipy.sparse matrix or array, got {type(matrix).__name__}.")
    if format.lower() != "csr":
        raise ValueError("format must be 'csr' in this build (CSC and COO are outside the path).")
    idt = _index_dtype(index_dtype)
    csr = matrix.tocsr(copy=True)
    if canonical:
        csr.sum_duplicates()
        csr.sort_indices()
    vdt = _numpy_value_dtype(np.asarray(csr.data), dtype)
    values = np.asarray(csr.data)
    if vdt == torch.bfloat16:
        data = torch.from_numpy(np.ascontiguousarray(values, dtype=np.float32)).to(torch.bfloat16)
    elif vdt == torch.complex64:
        data = torch.from_numpy(np.ascontiguousarray(values, dtype=np.complex64))
    elif vdt == torch.float16:
        data = torch.from_numpy(np.ascontiguousarray(values, dtype=np.float16))
    else:
        if np.iscomplexobj(values):
            raise TypeError("complex values need dtype complex64.")
        data = torch.from_numpy(np.ascontiguousarray(values, dtype=np.float32))
    np_idx = np.int32 if idt == torch.int32 else np.int64
    device = default_torch_device()
    return CSRArray(
        data=data.to(device),
        indices=torch.from_numpy(np.ascontiguousarray(csr.indices, dtype=np_idx)).to(device),
        indptr=torch.from_numpy(np.ascontiguousarray(csr.indptr, dtype=np_idx)).to(device),
        shape=tuple(int(s) for s in csr.shape),
        sorted_indices=bool(canonical),
        has_canonical_format=bool(canonical),
    )
