"""Native CPU adjoint entry points (msx_csr_transpose_cpu,
msx_csr_spmv/spmm_transpose_cpu, msx_csr_spmv/spmm_data_vjp_cpu) against the
oracle, bit for bit, through the C ABI: every value type, both index types,
one and several workers (the worker count changes the rounding of the
transposed products, as in the reference)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import _capi
from _util import TORCH, storage, to_numpy, to_torch

VTYPES = ["float32", "float16", "bfloat16", "complex64"]


def _case(rng, n_rows, n_cols, index_dtype, vtype, long_rows=True):
    lengths = rng.integers(0, 10, n_rows)
    lengths[rng.random(n_rows) < 0.15] = 0
    if long_rows:
        lengths[rng.random(n_rows) < 0.02] = 200
    indptr = np.zeros(n_rows + 1, np.int64)
    np.cumsum(lengths, out=indptr[1:])
    nnz = int(indptr[-1])
    indices = rng.integers(0, n_cols, nnz)
    vals = rng.standard_normal(nnz).astype(np.float32)
    if vtype == "complex64":
        vals = (vals + 1j * rng.standard_normal(nnz)).astype(np.complex64)
    return storage(vals, vtype), indices.astype(index_dtype), indptr.astype(index_dtype)


def _dense_operand(rng, shape, vtype):
    v = rng.standard_normal(shape).astype(np.float32)
    if vtype == "complex64":
        v = (v + 1j * rng.standard_normal(shape)).astype(np.complex64)
    return storage(v, vtype)


def _t(arr, vtype=None):
    return to_torch(arr, vtype)


def _bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint8)


@pytest.mark.parametrize("vtype", VTYPES)
@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_transpose_cpu_equals_oracle(oracle, vtype, index_dtype):
    rng = np.random.default_rng(7)
    data, ind, ptr = _case(rng, 500, 300, index_dtype, vtype)
    td, ti, tp = _capi.transpose(_t(data, vtype), _t(ind), _t(ptr), 500, 300)
    wd, wi, wp = oracle.csr_transpose(data, ind, ptr, 500, 300, vtype=vtype)
    np.testing.assert_array_equal(to_numpy(tp), wp)
    np.testing.assert_array_equal(to_numpy(ti), wi)
    np.testing.assert_array_equal(_bits(to_numpy(td)), _bits(wd))


@pytest.mark.parametrize("vtype", VTYPES)
def test_transpose_cpu_dropped_columns_tail(oracle, vtype):
    """Columns out of range are dropped from the transpose (the oracle's
    transpose holds t_indptr[n_cols] entries); the output buffers' tail past
    t_indptr[n_cols] holds zero bits and row 0 on the native CPU path, not
    whatever the buffers held."""
    rng = np.random.default_rng(3)
    data, ind, ptr = _case(rng, 400, 200, np.int32, vtype)
    ind = ind.copy()
    ind[[2, 50, 51]] = [200, 10_000, -4]
    nnz = int(ptr[-1])
    td, ti, tp = _capi.transpose(_t(data, vtype), _t(ind), _t(ptr), 400, 200)
    wd, wi, wp = oracle.csr_transpose(data, ind, ptr, 400, 200, vtype=vtype)
    kept = nnz - 3
    assert int(wp[-1]) == kept and len(wd) == kept
    np.testing.assert_array_equal(to_numpy(tp), wp)
    np.testing.assert_array_equal(to_numpy(ti)[:kept], wi)
    np.testing.assert_array_equal(_bits(to_numpy(td)[:kept]), _bits(wd))
    assert not _bits(to_numpy(td)[kept:]).any() and not to_numpy(ti)[kept:].any()


@pytest.mark.parametrize("vtype", VTYPES)
@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
@pytest.mark.parametrize("threads", [1, 3, 8])
def test_spmv_transpose_cpu_equals_oracle(oracle, vtype, index_dtype, threads):
    rng = np.random.default_rng(100 + threads)
    data, ind, ptr = _case(rng, 700, 350, index_dtype, vtype)
    x = _dense_operand(rng, 700, vtype)
    got = _capi.spmv_transpose(_t(data, vtype), _t(ind), _t(ptr), _t(x, vtype), 700, 350,
                               n_threads=threads)
    want = oracle.csr_transpose_product(data, ind, ptr, x, 700, 350, vtype=vtype,
                                        n_threads=threads)
    np.testing.assert_array_equal(_bits(to_numpy(got)), _bits(want))


@pytest.mark.parametrize("vtype", VTYPES)
@pytest.mark.parametrize("threads", [1, 4])
@pytest.mark.parametrize("k", [1, 3, 16])
def test_spmm_transpose_cpu_equals_oracle(oracle, vtype, threads, k):
    rng = np.random.default_rng(200 + k)
    data, ind, ptr = _case(rng, 400, 260, np.int32, vtype)
    X = _dense_operand(rng, (400, k), vtype)
    got = _capi.spmm_transpose(_t(data, vtype), _t(ind), _t(ptr), _t(X, vtype), 400, 260,
                               n_threads=threads)
    want = oracle.csr_transpose_product(data, ind, ptr, X, 400, 260, vtype=vtype,
                                        n_threads=threads)
    np.testing.assert_array_equal(_bits(to_numpy(got)), _bits(want))


def test_transpose_product_partition_order_native(oracle):
    # the grouping case that separates one worker from two
    e = np.float32(2.0 ** -24)
    data = np.array([1.0, 0.0, e, e], np.float32)
    ind = np.array([0, 1, 0, 0], np.int32)
    ptr = np.array([0, 2, 4], np.int32)
    x = np.ones(2, np.float32)
    for threads, want in ((1, 1.0), (2, 1.0 + 2.0 ** -23)):
        got = _capi.spmv_transpose(_t(data), _t(ind), _t(ptr), _t(x), 2, 2, n_threads=threads)
        assert got[0].item() == want


@pytest.mark.parametrize("vtype", VTYPES)
@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_data_vjp_cpu_equals_oracle(oracle, vtype, index_dtype):
    rng = np.random.default_rng(300)
    data, ind, ptr = _case(rng, 450, 210, index_dtype, vtype)
    nnz = data.size
    x = _dense_operand(rng, 210, vtype)
    cot = _dense_operand(rng, 450, vtype)
    for threads in (1, 5):
        got = _capi.spmv_data_vjp(_t(ind), _t(ptr), _t(x, vtype), _t(cot, vtype), 450, 210,
                                  n_threads=threads)
        want = oracle.csr_data_vjp(ind, ptr, x, cot, 450, 210, nnz, vtype=vtype)
        np.testing.assert_array_equal(_bits(to_numpy(got)), _bits(want))
    for k in (1, 4, 33):
        X = _dense_operand(rng, (210, k), vtype)
        C = _dense_operand(rng, (450, k), vtype)
        got = _capi.spmm_data_vjp(_t(ind), _t(ptr), _t(X, vtype), _t(C, vtype), 450, 210,
                                  n_threads=3)
        want = oracle.csr_data_vjp(ind, ptr, X, C, 450, 210, nnz, vtype=vtype)
        np.testing.assert_array_equal(_bits(to_numpy(got)), _bits(want))


def test_adjoint_edge_cases_cpu(oracle):
    f = torch.float32
    empty_i = torch.zeros(0, dtype=torch.int32)
    # zero rows: A^T x is all zeros; transpose of a 0 x 4 matrix
    y = _capi.spmv_transpose(torch.zeros(0, dtype=f), empty_i, torch.zeros(1, dtype=torch.int32),
                             torch.zeros(0, dtype=f), 0, 4, n_threads=4)
    assert torch.equal(y, torch.zeros(4))
    td, ti, tp = _capi.transpose(torch.zeros(0, dtype=f), empty_i,
                                 torch.zeros(1, dtype=torch.int32), 0, 4)
    assert tp.tolist() == [0] * 5
    # zero columns
    y = _capi.spmv_transpose(torch.zeros(0, dtype=f), empty_i, torch.zeros(4, dtype=torch.int32),
                             torch.ones(3), 3, 0)
    assert y.numel() == 0
    # all rows empty, k = 0
    Y = _capi.spmm_transpose(torch.zeros(0, dtype=f), empty_i, torch.zeros(4, dtype=torch.int32),
                             torch.ones(3, 0), 3, 2)
    assert Y.shape == (2, 0)
    g = _capi.spmm_data_vjp(torch.tensor([1], dtype=torch.int32),
                            torch.tensor([0, 1], dtype=torch.int32), torch.ones(2, 0),
                            torch.ones(1, 0), 1, 2)
    assert g.tolist() == [0.0]


def test_adjoint_cpu_rejects_bad_arguments():
    f = torch.float32
    ptr = torch.tensor([0, 1], dtype=torch.int32)
    ind = torch.tensor([0], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="-?[1-9]"):
        _capi.spmv_transpose(torch.ones(1, dtype=f), ind, ptr, torch.ones(1), -1, 1)
    L = _capi.lib()
    st = L.msx_csr_transpose_cpu(9, 0, 1, 1, 1, ind.data_ptr(), ind.data_ptr(), ptr.data_ptr(),
                                 ind.data_ptr(), ind.data_ptr(), ptr.data_ptr())
    assert st != _capi.OK and _capi.last_error()
