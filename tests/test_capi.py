"""The C-ABI library loads, exports every declared entry point, and rejects
bad arguments with the documented status codes (no GPU needed: checks run
before any HIP call)."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import _capi


def test_exports_every_declared_symbol():
    names = _capi.declared_functions()
    assert len(names) >= 12, names
    L = _capi.lib()
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_abi_version():
    assert _capi.lib().msx_abi_version() == 7


def _f32(a):
    return np.ascontiguousarray(a, np.float32)


def test_cpu_entry_point_kat():
    d = _f32([2, -1, 4, 5])
    i = np.array([0, 2, 1, 3], np.int32)
    p = np.array([0, 2, 2, 4], np.int32)
    x = _f32([3, 10, 7, -2])
    y = np.zeros(3, np.float32)
    L = _capi.lib()
    st = L.msx_csr_spmv_cpu(0, 0, 3, 4, 4, d.ctypes.data, i.ctypes.data, p.ctypes.data,
                            x.ctypes.data, y.ctypes.data, 2)
    assert st == _capi.OK
    np.testing.assert_array_equal(y, [-1, 0, 30])
    X = _f32([[3, 1], [10, -2], [7, 4], [-2, 6]])
    Y = np.zeros((3, 2), np.float32)
    st = L.msx_csr_spmm_cpu(0, 0, 3, 4, 4, d.ctypes.data, i.ctypes.data, p.ctypes.data, 2,
                            X.ctypes.data, Y.ctypes.data, 1)
    assert st == _capi.OK
    np.testing.assert_array_equal(Y, [[-1, -2], [0, 0], [30, 22]])


@pytest.mark.parametrize("fn", ["msx_csr_spmv", "msx_csr_spmv_cpu"])
def test_argument_errors(fn):
    L = _capi.lib()
    dummy = ctypes.c_void_p(16)
    f = getattr(L, fn)
    tail = [None] if fn == "msx_csr_spmv" else [1]
    extra = [None] if fn == "msx_csr_spmv" else []
    def call(vt, it, n_rows, n_cols, nnz, indptr=dummy):
        return f(vt, it, n_rows, n_cols, nnz, dummy, dummy, indptr, dummy, dummy, *extra, *tail)
    assert call(9, 0, 1, 1, 1) == _capi.ETYPE
    assert "dtype" in _capi.last_error()
    assert call(0, 5, 1, 1, 1) == _capi.ETYPE
    assert "int32 or int64" in _capi.last_error()
    assert call(0, 0, -1, 1, 1) == _capi.EINVAL
    assert "non-negative" in _capi.last_error()
    assert call(0, 0, 1, 1, 1, indptr=None) == _capi.EINVAL


def test_plan_rejects_bad_block_nnz():
    L = _capi.lib()
    out = ctypes.c_void_p()
    st = L.msx_csr_plan_create(0, 4, 4, ctypes.c_void_p(16), 100, None, ctypes.byref(out))
    assert st == _capi.EINVAL and "block_nnz" in _capi.last_error()
    st = L.msx_csr_plan_create(3, 4, 4, ctypes.c_void_p(16), 0, None, ctypes.byref(out))
    assert st == _capi.ETYPE


def test_spmm_rejects_short_leading_dimension():
    L = _capi.lib()
    d = ctypes.c_void_p(16)
    st = L.msx_csr_spmm(0, 0, 2, 2, 2, d, d, d, 4, d, 3, d, 4, None, None)
    assert st == _capi.EINVAL and "leading" in _capi.last_error()


def test_cpu_ranges_entry_point():
    L = _capi.lib()
    work = np.array([5, 1, 1, 1, 9, 2], np.int64)
    out = np.zeros(8, np.int64)
    n = ctypes.c_int64()
    assert L.msx_cpu_ranges(work.ctypes.data, 6, 4, out.ctypes.data, ctypes.byref(n)) == _capi.OK
    ranges = out[: 2 * n.value].reshape(-1, 2)
    assert ranges[0, 0] == 0 and ranges[-1, 1] == 6
    assert np.all(ranges[1:, 0] == ranges[:-1, 1])


def test_transpose_layout_argument_errors():
    """The two-pass regather's entry points check their arguments before any
    HIP call: value type, nnz range, NULL buffers; nnz = 0 is a no-op."""
    L = _capi.lib()
    d = ctypes.c_void_p(16)
    assert L.msx_csr_transpose_layout(9, 10, d, d, d, d, None) == _capi.ETYPE
    assert L.msx_csr_transpose_layout(0, -1, d, d, d, d, None) == _capi.EINVAL
    assert L.msx_csr_transpose_layout(0, 1 << 31, d, d, d, d, None) == _capi.EINVAL
    assert L.msx_csr_transpose_layout(0, 10, None, d, d, d, None) == _capi.EINVAL
    assert L.msx_csr_transpose_layout(0, 10, d, d, None, d, None) == _capi.EINVAL
    assert L.msx_csr_transpose_layout(0, 0, None, None, None, None, None) == _capi.OK
    f = L.msx_csr_transpose_values_layout
    assert f(9, 10, d, d, d, d, 0, d, d, None) == _capi.ETYPE
    assert f(0, -1, d, d, d, d, 0, d, d, None) == _capi.EINVAL
    assert f(0, 10, d, d, d, d, 0, None, d, None) == _capi.EINVAL
    assert f(3, 10, d, d, d, d, 1, d, None, None) == _capi.EINVAL
    assert f(0, 0, None, None, None, None, 0, None, None, None) == _capi.OK
