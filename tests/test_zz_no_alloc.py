"""msx_csr_spmv_transpose_noalloc: the transposed SpMV without any
allocation (16-bit values accumulate in the library's fixed device scratch
array), checked through the C ABI against msx_csr_spmv_transpose, the
allocating entry point, on two calls in a row, the second with a smaller
matrix (the scratch keeps the first call's contents and must be cleared).

Small-integer values make every float32 sum exact whatever the order of the
atomic additions, so both entry points must agree bit for bit; normal values
agree within the path's tolerance, 1e-2 (16-bit) / 1e-5 (float32,
complex64) times sum |a_ij x_i| per output, and with the oracle.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import _capi
from _util import TOL, assert_rows_close, storage, to_numpy, to_torch
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

DEV = "cuda"
VTYPES = ["float16", "bfloat16", "float32", "complex64"]


def _matrix(rng, n_rows, n_cols, max_len):
    lengths = rng.integers(0, max_len, n_rows)
    indptr = np.zeros(n_rows + 1, np.int64)
    np.cumsum(lengths, out=indptr[1:])
    indices = rng.integers(0, n_cols, int(indptr[-1]))
    return indices.astype(np.int32), indptr.astype(np.int32)


def _noalloc(d, i, p, x, n_rows, n_cols):
    y = torch.full((n_cols,), float("nan"), dtype=d.dtype, device=DEV)
    st = _capi.lib().msx_csr_spmv_transpose_noalloc(
        _capi.VT[d.dtype], _capi.IT[i.dtype], n_rows, n_cols, d.numel(), d.data_ptr(),
        i.data_ptr(), p.data_ptr(), x.data_ptr(), y.data_ptr(), _capi._stream())
    if st != _capi.OK:
        raise RuntimeError(f"msx_csr_spmv_transpose_noalloc: {st} {_capi.last_error()}")
    return y


def _values(rng, n, vtype, integers):
    if integers:
        v = rng.integers(-2, 3, n).astype(np.float64)
        if vtype == "complex64":
            v = v + 1j * rng.integers(-2, 3, n)
    else:
        v = rng.standard_normal(n)
        if vtype == "complex64":
            v = v + 1j * rng.standard_normal(n)
    return storage(v, vtype)


@pytest.mark.parametrize("vtype", VTYPES)
def test_noalloc_matches_the_allocating_entry_point(vtype):
    rng = np.random.default_rng(61)
    for n_rows, n_cols in ((60_000, 50_000), (900, 700)):  # second call smaller
        indices, indptr = _matrix(rng, n_rows, n_cols, 24)
        nnz = int(indptr[-1])
        i, p = to_torch(indices, None, DEV), to_torch(indptr, None, DEV)
        for integers in (True, False):
            data, x = _values(rng, nnz, vtype, integers), _values(rng, n_rows, vtype, integers)
            d, xt = to_torch(data, vtype, DEV), to_torch(x, vtype, DEV)
            got = to_numpy(_noalloc(d, i, p, xt, n_rows, n_cols))
            ref = to_numpy(_capi.spmv_transpose(d, i, p, xt, n_rows, n_cols))
            torch.cuda.synchronize()
            what = f"{vtype} {n_rows}x{n_cols} {'integers' if integers else 'normal'}"
            if integers:
                np.testing.assert_array_equal(got, ref, err_msg=what)
            td, ti, tp = orc.csr_transpose(data, indices, indptr, n_rows, n_cols, vtype=vtype)
            want = orc.csr_matvec(td, ti, tp, x, n_cols, vtype=vtype)
            scale = orc.row_scale(td, ti, tp, x, n_cols, vtype=vtype)
            assert_rows_close(got, ref, scale, vtype, f"{what} vs allocating entry point")
            assert_rows_close(got, want, scale, vtype, f"{what} vs oracle")


def test_noalloc_rejects_sizes_beyond_its_scratch():
    d = torch.zeros(1, dtype=torch.float16, device=DEV)
    i = torch.zeros(1, dtype=torch.int32, device=DEV)
    p = torch.tensor([0, 1], dtype=torch.int32, device=DEV)
    x = torch.zeros(1, dtype=torch.float16, device=DEV)
    y = torch.zeros(1, dtype=torch.float16, device=DEV)
    n_cols = (1 << 23) + 1
    st = _capi.lib().msx_csr_spmv_transpose_noalloc(
        _capi.VT[torch.float16], 0, 1, n_cols, 1, d.data_ptr(), i.data_ptr(), p.data_ptr(),
        x.data_ptr(), y.data_ptr(), _capi._stream())
    assert st == _capi.EINVAL
    assert "8388608" in _capi.last_error()
