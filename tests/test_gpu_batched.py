"""HIP batched SpMV / SpMM parity with the CPU oracle, through the C ABI and
the drop-in API.

The reference's batched kernels sum every output from zero in stored order
(reference: src/sparse/csr_batched_matvec/csr_batched_matvec.cpp:82-146,
src/sparse/csr_batched_matmul/csr_batched_matmul.cpp:85-248), as the HIP
SpMM does, so every value type must equal the oracle bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import _capi
from _util import storage, to_numpy, to_torch
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

DEV = "cuda"
VTYPES = ["float32", "float16", "bfloat16", "complex64"]


def _values(rng, shape, vtype):
    v = rng.standard_normal(shape)
    if vtype == "complex64":
        v = v + 1j * rng.standard_normal(shape)
    return storage(v, vtype)


def _matrix(rng, n_rows, n_cols, index_dtype):
    lengths = rng.integers(0, 30, n_rows)
    lengths[rng.random(n_rows) < 0.1] = 0
    lengths[[0, n_rows // 2]] = [700, 2500]  # long rows
    indptr = np.zeros(n_rows + 1, np.int64)
    np.cumsum(lengths, out=indptr[1:])
    nnz = int(indptr[-1])
    return rng.integers(0, n_cols, nnz).astype(index_dtype), indptr.astype(index_dtype), nnz


def _want_vectors(data, indices, indptr, X, n_rows, vtype):
    return np.ascontiguousarray(
        orc.csr_matmul(data, indices, indptr, np.ascontiguousarray(X.T), n_rows, vtype=vtype).T)


def _bytes(a):
    return np.ascontiguousarray(a).view(np.uint8)


@pytest.mark.parametrize("vtype", VTYPES)
@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_batched_spmv_parity_and_strides(vtype, index_dtype):
    rng = np.random.default_rng(5)
    n_rows, n_cols = 1500, 1200
    indices, indptr, nnz = _matrix(rng, n_rows, n_cols, index_dtype)
    data = _values(rng, nnz, vtype)
    d, i, p = (to_torch(a, vtype if a is data else None, DEV) for a in (data, indices, indptr))
    for batch in (1, 2, 3, 8, 16, 17, 32):  # 16-byte vectors per column: 1, 2, 4, 8 and others
        X = _values(rng, (batch, n_cols + 5), vtype)  # row stride n_cols + 5
        want = _want_vectors(data, indices, indptr, np.ascontiguousarray(X[:, :n_cols]), n_rows,
                             vtype)
        Xt = to_torch(X, vtype, DEV)
        Y = torch.zeros((batch, n_rows + 3), dtype=Xt.dtype, device=DEV)
        Y[:, n_rows:] = 2
        _capi.batched_spmv(d, i, p, Xt, n_rows, n_cols, Y=Y, ldx=n_cols + 5, ldy=n_rows + 3)
        torch.cuda.synchronize()
        assert torch.all(Y[:, n_rows:] == 2)  # row padding untouched
        got = to_numpy(Y)[:, :n_rows]
        np.testing.assert_array_equal(_bytes(got), _bytes(want), err_msg=f"{vtype} batch={batch}")


@pytest.mark.parametrize("vtype", VTYPES)
def test_batched_spmm_parity_and_batch_strides(vtype):
    rng = np.random.default_rng(6)
    n_rows, n_cols = 900, 700
    indices, indptr, nnz = _matrix(rng, n_rows, n_cols, np.int32)
    data = _values(rng, nnz, vtype)
    d, i, p = (to_torch(a, vtype if a is data else None, DEV) for a in (data, indices, indptr))
    per16 = 16 // storage(np.zeros(1), vtype).itemsize
    line_k = 256 // storage(np.zeros(1), vtype).itemsize  # X rows of two cache lines
    for batch, k in ((1, 4), (3, 1), (3, 7), (2, 2 * per16), (4, line_k)):
        full = _values(rng, (batch, n_cols + 2, k), vtype)  # batch stride (n_cols + 2) * k
        Xt = to_torch(full, vtype, DEV)[:, :n_cols, :]
        want = np.stack([orc.csr_matmul(data, indices, indptr, np.ascontiguousarray(full[b, :n_cols]),
                                        n_rows, vtype=vtype) for b in range(batch)])
        Y = _capi.batched_spmm(d, i, p, Xt, n_rows, n_cols)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_bytes(to_numpy(Y)), _bytes(want),
                                      err_msg=f"{vtype} batch={batch} k={k}")


def test_batches_beyond_one_launch():
    # more batches than one launch's grid y extent (65535)
    data = np.array([1.0, 2.0, -3.0], np.float32)
    indices = np.array([0, 1, 1], np.int32)
    indptr = np.array([0, 2, 2, 3], np.int32)
    d, i, p = (to_torch(a, None, DEV) for a in (data, indices, indptr))
    batch = 70_000
    X = np.random.default_rng(7).standard_normal((batch, 2)).astype(np.float32)
    Xt = to_torch(X, None, DEV)
    want = _want_vectors(data, indices, indptr, X, 3, "float32")
    got = to_numpy(_capi.batched_spmv(d, i, p, Xt, 3, 2))
    np.testing.assert_array_equal(got, want)
    got = to_numpy(_capi.batched_spmm(d, i, p, Xt.reshape(batch, 2, 1), 3, 2))
    np.testing.assert_array_equal(got[:, :, 0], want)


def test_batched_through_api(gpu):
    rng = np.random.default_rng(8)
    indices, indptr, nnz = _matrix(rng, 400, 300, np.int64)
    data = rng.standard_normal(nnz).astype(np.float32)
    A = gpu.csr_array((data, indices, indptr), shape=(400, 300))
    V = rng.standard_normal((2, 5, 300)).astype(np.float32)
    M = rng.standard_normal((3, 300, 6)).astype(np.float32)
    yv = gpu.csr_batched_matvec(A, torch.from_numpy(V).to(DEV))
    ym = gpu.csr_batched_matmul(A, torch.from_numpy(M).to(DEV))
    assert yv.shape == (2, 5, 400) and ym.shape == (3, 400, 6) and yv.is_cuda
    np.testing.assert_array_equal(yv.cpu().numpy().reshape(10, 400),
                                  _want_vectors(data, indices, indptr, V.reshape(10, 300), 400,
                                                "float32"))
    np.testing.assert_array_equal(
        ym.cpu().numpy(), np.stack([orc.csr_matmul(data, indices, indptr, M[b], 400) for b in range(3)]))
    np.testing.assert_array_equal((A @ torch.from_numpy(M).to(DEV)).cpu().numpy(), ym.cpu().numpy())
