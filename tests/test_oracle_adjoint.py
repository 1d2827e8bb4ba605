"""Pins the adjoint side of the CPU oracle (oracle/csr_oracle.c:
oracle_csr_transpose, oracle_csr_transpose_product, oracle_csr_data_vjp)
before it checks the native and HIP paths.

A dropped term, a transposed operand or a wrong index fails at least one of:
SciPy's CSR->CSC conversion (the same stable counting sort), dense float64
brute force on small integers (where float32 sums are exact), the adjoint
identity <A x, y> = <x, A^T y>, the reference's gradient known answers
(tests/test_grad.py:28-221), a grouping case on which the reference's
per-range partial sums and a sequential sum round differently, and the
sign-of-zero rule that tells the one-product SpMV value gradient from the
summed SpMM one.
"""

from __future__ import annotations

import numpy as np
import pytest

from _util import storage, widen

KAT_DATA = np.array([2.0, -1.0, 4.0, 5.0], np.float32)
KAT_IND = np.array([0, 2, 1, 3], np.int32)
KAT_PTR = np.array([0, 2, 2, 4], np.int32)
KAT_ROWS = np.array([0, 0, 2, 2])


def _dense(data, indices, indptr, shape, dtype=np.float64):
    A = np.zeros(shape, dtype)
    for r in range(shape[0]):
        for p in range(int(indptr[r]), int(indptr[r + 1])):
            A[r, int(indices[p])] += data[p]
    return A


def _random(rng, n_rows, n_cols, *, integer=True, index_dtype=np.int32, max_len=9,
            dup=False):
    lengths = rng.integers(0, max_len, n_rows)
    lengths[rng.random(n_rows) < 0.1] = 0
    indptr = np.zeros(n_rows + 1, np.int64)
    np.cumsum(lengths, out=indptr[1:])
    nnz = int(indptr[-1])
    if dup:
        indices = rng.integers(0, n_cols, nnz)
    else:
        indices = np.concatenate([np.sort(rng.choice(n_cols, size=min(int(n), n_cols),
                                                     replace=False)) for n in lengths]
                                 ).astype(np.int64) if nnz else np.zeros(0, np.int64)
        indptr = np.zeros(n_rows + 1, np.int64)
        np.cumsum(np.minimum(lengths, n_cols), out=indptr[1:])
        nnz = int(indptr[-1])
    data = (rng.integers(-4, 5, nnz) if integer else rng.standard_normal(nnz)).astype(np.float32)
    return data, indices.astype(index_dtype), indptr.astype(index_dtype)


# -- transpose -----------------------------------------------------------------

@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_transpose_matches_scipy_tocsc(oracle, index_dtype):
    import scipy.sparse as sp

    rng = np.random.default_rng(11)
    data, ind, ptr = _random(rng, 300, 170, integer=False, index_dtype=index_dtype, dup=True)
    td, ti, tp = oracle.csr_transpose(data, ind, ptr, 300, 170)
    S = sp.csr_matrix((data, ind, ptr), shape=(300, 170))
    C = S.tocsc()  # csr_tocsc: per-column counting sort, stable in row order
    np.testing.assert_array_equal(tp, C.indptr)
    np.testing.assert_array_equal(ti, C.indices)
    np.testing.assert_array_equal(td, C.data)
    assert ti.dtype == index_dtype and tp.dtype == index_dtype


def test_transpose_kat_and_dense(oracle):
    # reference tests/test_transpose.py:23-36
    td, ti, tp = oracle.csr_transpose(KAT_DATA, KAT_IND, KAT_PTR, 3, 4)
    np.testing.assert_array_equal(tp, [0, 1, 2, 3, 4])
    np.testing.assert_array_equal(ti, [0, 2, 0, 2])
    np.testing.assert_array_equal(td, [2.0, 4.0, -1.0, 5.0])
    np.testing.assert_array_equal(_dense(td, ti, tp, (4, 3)),
                                  _dense(KAT_DATA, KAT_IND, KAT_PTR, (3, 4)).T)


def test_transpose_edge_cases(oracle):
    # no rows, no columns, empty rows
    td, ti, tp = oracle.csr_transpose(np.zeros(0, np.float32), np.zeros(0, np.int32),
                                      np.zeros(1, np.int32), 0, 5)
    np.testing.assert_array_equal(tp, np.zeros(6))
    td, ti, tp = oracle.csr_transpose(np.zeros(0, np.float32), np.zeros(0, np.int32),
                                      np.zeros(4, np.int32), 3, 0)
    np.testing.assert_array_equal(tp, [0])
    # bfloat16 / complex values move as bit patterns
    bits = np.array([0x3F80, 0x8000, 0x7FC1], np.uint16)
    td, _, _ = oracle.csr_transpose(bits, np.array([2, 0, 1], np.int32),
                                    np.array([0, 3], np.int32), 1, 3, vtype="bfloat16")
    np.testing.assert_array_equal(td, [0x8000, 0x7FC1, 0x3F80])
    c = np.array([1 + 2j, -3j], np.complex64)
    td, _, _ = oracle.csr_transpose(c, np.array([1, 0], np.int32), np.array([0, 1, 2], np.int32),
                                    2, 2)
    np.testing.assert_array_equal(td, [-3j, 1 + 2j])


# -- transposed products -------------------------------------------------------

@pytest.mark.parametrize("threads", [1, 3, 8])
@pytest.mark.parametrize("k", [None, 1, 5])
def test_transpose_product_exact_on_integers(oracle, threads, k):
    rng = np.random.default_rng(5 + threads)
    data, ind, ptr = _random(rng, 400, 260, dup=True)
    A = _dense(data, ind, ptr, (400, 260))
    X = rng.integers(-4, 5, 400 if k is None else (400, k)).astype(np.float32)
    got = oracle.csr_transpose_product(data, ind, ptr, X, 400, 260, n_threads=threads)
    np.testing.assert_array_equal(got.astype(np.float64), A.T @ X.astype(np.float64))


@pytest.mark.parametrize("vtype", ["float32", "complex64"])
def test_adjoint_identity(oracle, vtype):
    rng = np.random.default_rng(17)
    data, ind, ptr = _random(rng, 500, 333, integer=False, dup=True)
    if vtype == "complex64":
        data = (data + 1j * rng.standard_normal(data.size)).astype(np.complex64)
    x = rng.standard_normal(333).astype(np.float32)
    y = rng.standard_normal(500).astype(np.float32)
    if vtype == "complex64":
        x = (x + 1j * rng.standard_normal(333)).astype(np.complex64)
        y = (y + 1j * rng.standard_normal(500)).astype(np.complex64)
    Ax = oracle.csr_matvec(data, ind, ptr, x, 500).astype(np.complex128)
    Aty = oracle.csr_transpose_product(data, ind, ptr, y, 500, 333).astype(np.complex128)
    lhs = np.sum(Ax * y)  # bilinear pairing: no conjugation on either side
    rhs = np.sum(x * Aty)
    scale = np.sum(np.abs(_dense(np.abs(data), ind, ptr, (500, 333)))
                   * np.abs(y)[:, None] * np.abs(x)[None, :])
    assert abs(lhs - rhs) <= 1e-5 * scale


def test_transpose_product_equals_transpose_then_spmv_on_single_entry_columns(oracle):
    # every column holds at most one value: A^T x has one product per output,
    # so both routes round once and must agree bit for bit
    rng = np.random.default_rng(3)
    n_rows, n_cols = 90, 120
    cols = rng.permutation(n_cols)[:80]
    rows = np.sort(rng.integers(0, n_rows, 80))
    ptr = np.searchsorted(rows, np.arange(n_rows + 1)).astype(np.int32)
    ind = cols.astype(np.int32)
    data = rng.standard_normal(80).astype(np.float32)
    x = rng.standard_normal(n_rows).astype(np.float32)
    td, ti, tp = oracle.csr_transpose(data, ind, ptr, n_rows, n_cols)
    want = oracle.csr_matvec(td, ti, tp, x, n_cols)
    got = oracle.csr_transpose_product(data, ind, ptr, x, n_rows, n_cols)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_transpose_product_partition_order(oracle):
    # rows of equal work -> ranges [0,1), [1,2) with two workers
    # (equal_cpu_ranges, reference cpu_parallel.h:160-162).  Column 0 gets
    # 1.0 from row 0 and 2^-24 twice from row 1.  One worker: (1 + e) + e
    # rounds to 1 twice.  Two workers: partial 1 = e + e = 2^-23, then
    # 0 + 1 + 2^-23 = 1 + 2^-23 exactly.
    assert oracle.cpu_ranges([2, 2], 2) == [(0, 1), (1, 2)]
    e = np.float32(2.0 ** -24)
    data = np.array([1.0, 0.0, e, e], np.float32)
    ind = np.array([0, 1, 0, 0], np.int32)
    ptr = np.array([0, 2, 4], np.int32)
    x = np.ones(2, np.float32)
    one = oracle.csr_transpose_product(data, ind, ptr, x, 2, 2, n_threads=1)
    two = oracle.csr_transpose_product(data, ind, ptr, x, 2, 2, n_threads=2)
    assert one[0] == np.float32(1.0)
    assert two[0] == np.float32(1.0 + 2.0 ** -23)
    X = np.ones((2, 3), np.float32)
    two_m = oracle.csr_transpose_product(data, ind, ptr, X, 2, 2, n_threads=2)
    assert np.all(two_m[0] == np.float32(1.0 + 2.0 ** -23))


@pytest.mark.parametrize("vtype", ["float16", "bfloat16"])
def test_transpose_product_low_precision_rounds_once(oracle, vtype):
    # float32 accumulation then one rounding: values that are exact in the
    # storage type and sums that are exact in float32
    rng = np.random.default_rng(23)
    data, ind, ptr = _random(rng, 200, 140, dup=True)
    x = rng.integers(-4, 5, 200).astype(np.float32)
    A = _dense(data, ind, ptr, (200, 140))
    want = storage((A.T @ x.astype(np.float64)).astype(np.float32), vtype)
    got = oracle.csr_transpose_product(storage(data, vtype), ind, ptr, storage(x, vtype), 200,
                                       140, vtype=vtype)
    np.testing.assert_array_equal(got, want)
    # and a sum that is not exact in the storage type is rounded from float32
    d = storage(np.array([1.0, 2.0 ** -9, 2.0 ** -9], np.float32), vtype)
    got = oracle.csr_transpose_product(d, np.zeros(3, np.int32), np.array([0, 1, 2, 3], np.int32),
                                       storage(np.ones(3, np.float32), vtype), 3, 1, vtype=vtype)
    exact = np.float32(1.0 + 2.0 ** -8)
    np.testing.assert_array_equal(got, storage(np.array([exact]), vtype))


def test_transpose_product_complex_against_numpy(oracle):
    rng = np.random.default_rng(29)
    data, ind, ptr = _random(rng, 150, 90, dup=True)
    data = (data + 1j * rng.integers(-4, 5, data.size)).astype(np.complex64)
    X = (rng.integers(-4, 5, (150, 3)) + 1j * rng.integers(-4, 5, (150, 3))).astype(np.complex64)
    A = _dense(data, ind, ptr, (150, 90), np.complex128)
    got = oracle.csr_transpose_product(data, ind, ptr, X, 150, 90, n_threads=4)
    np.testing.assert_array_equal(got.astype(np.complex128), A.T @ X.astype(np.complex128))


# -- value gradients -----------------------------------------------------------

def test_data_vjp_reference_kat(oracle):
    # reference tests/test_grad.py:180-221: loss = sum((A x)^2), so
    # d loss / d a_p = 2 (A x)[row] * x[col]
    x = np.array([3.0, 10.0, 7.0, -2.0], np.float32)
    y = oracle.csr_matvec(KAT_DATA, KAT_IND, KAT_PTR, x, 3)
    g = oracle.csr_data_vjp(KAT_IND, KAT_PTR, x, 2 * y, 3, 4, 4)
    np.testing.assert_array_equal(g, 2 * y[KAT_ROWS] * x[KAT_IND])
    np.testing.assert_array_equal(g, [-6.0, -14.0, 600.0, -120.0])


@pytest.mark.parametrize("k", [1, 4])
def test_data_vjp_matches_dense_gradient(oracle, k):
    # d/dA of <C, A X> is C X^T, sampled at the stored coordinates; integer
    # operands keep every float32 sum exact
    rng = np.random.default_rng(31 + k)
    data, ind, ptr = _random(rng, 120, 80)
    rows = np.repeat(np.arange(120), np.diff(ptr))
    X = rng.integers(-4, 5, (80, k)).astype(np.float32)
    C = rng.integers(-4, 5, (120, k)).astype(np.float32)
    dense = C.astype(np.float64) @ X.T.astype(np.float64)
    got = oracle.csr_data_vjp(ind, ptr, X, C, 120, 80, data.size)
    np.testing.assert_array_equal(got.astype(np.float64), dense[rows, ind])
    # finite difference of the bilinear form, one coordinate
    p = data.size // 2
    bump = data.copy()
    bump[p] += 1.0
    f0 = np.sum(C * oracle.csr_matmul(data, ind, ptr, X, 120))
    f1 = np.sum(C * oracle.csr_matmul(bump, ind, ptr, X, 120))
    assert f1 - f0 == got[p]


def test_data_vjp_single_product_and_sign_of_zero(oracle):
    # SpMV rule: one product, so (-1) * 0 keeps its sign; SpMM rule sums
    # from +0, so the same product at k = 1 becomes +0
    ind = np.array([0], np.int32)
    ptr = np.array([0, 1], np.int32)
    x = np.array([0.0], np.float32)
    cot = np.array([-1.0], np.float32)
    g1 = oracle.csr_data_vjp(ind, ptr, x, cot, 1, 1, 1)
    gk = oracle.csr_data_vjp(ind, ptr, x.reshape(1, 1), cot.reshape(1, 1), 1, 1, 1)
    assert np.signbit(g1[0]) and not np.signbit(gk[0])
    # one product rounds once: float32 product of float32 inputs
    rng = np.random.default_rng(37)
    data, ind, ptr = _random(rng, 60, 50, integer=False)
    rows = np.repeat(np.arange(60), np.diff(ptr))
    x = rng.standard_normal(50).astype(np.float32)
    cot = rng.standard_normal(60).astype(np.float32)
    got = oracle.csr_data_vjp(ind, ptr, x, cot, 60, 50, data.size)
    np.testing.assert_array_equal(got, (cot[rows].astype(np.float64)
                                        * x[ind].astype(np.float64)).astype(np.float32))


@pytest.mark.parametrize("vtype", ["float16", "bfloat16", "complex64"])
def test_data_vjp_other_types(oracle, vtype):
    rng = np.random.default_rng(41)
    data, ind, ptr = _random(rng, 70, 40)
    rows = np.repeat(np.arange(70), np.diff(ptr))
    X = rng.integers(-4, 5, (40, 3)).astype(np.float32)
    C = rng.integers(-4, 5, (70, 3)).astype(np.float32)
    if vtype == "complex64":
        X = (X + 1j * rng.integers(-4, 5, X.shape)).astype(np.complex64)
        C = (C + 1j * rng.integers(-4, 5, C.shape)).astype(np.complex64)
        want = np.sum(C[rows] * X[ind], axis=1).astype(np.complex64)
        got = oracle.csr_data_vjp(ind, ptr, X, C, 70, 40, data.size)
        np.testing.assert_array_equal(got, want)
        return
    want = storage(np.sum(C[rows] * X[ind], axis=1), vtype)
    got = oracle.csr_data_vjp(ind, ptr, storage(X, vtype), storage(C, vtype), 70, 40, data.size,
                              vtype=vtype)
    np.testing.assert_array_equal(widen(got, vtype), widen(want, vtype))
