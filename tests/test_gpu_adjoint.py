"""HIP adjoint path (transpose, transposed products, value gradients) against
the CPU oracle, through the C ABI.

- msx_csr_transpose is a pure data movement: bit-exact for every type.
- msx_csr_spmv/spmm_data_vjp compute each value's gradient in a fixed order:
  bit-exact.
- msx_csr_spmv/spmm_transpose scatter with float atomics (as the reference's
  GPU kernel does, csr_matvec_transpose.metal:27-49), so the order of the
  additions is free: bit-exact where every partial sum is exact (small
  integers), else within |got - want| <= tol * sum_i |a_ij x_i| per output
  (tol 1e-5 float32/complex64, 1e-2 float16/bfloat16: one rounding of a
  float32 sum).
- The deterministic route, transpose then the zero-start SpMM with k = 1,
  equals the reference's one-worker transposed product bit for bit.
- At the headline size (random 16 per row, 2^22 rows) the adjoint identity
  <A x, y> = <x, A^T y> holds within float32 rounding.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import _capi
from _util import TOL, storage, to_numpy, to_torch, widen
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

DEV = "cuda"
VTYPES = ["float32", "float16", "bfloat16", "complex64"]


def _matrix(rng, n_rows, n_cols, index_dtype, long_rows=True):
    lengths = rng.integers(0, 24, n_rows)
    lengths[rng.random(n_rows) < 0.1] = 0
    if long_rows and n_rows > 4:
        lengths[[1, n_rows // 2]] = [900, 3000]
    indptr = np.zeros(n_rows + 1, np.int64)
    np.cumsum(lengths, out=indptr[1:])
    nnz = int(indptr[-1])
    return rng.integers(0, n_cols, nnz).astype(index_dtype), indptr.astype(index_dtype), nnz


def _values(rng, shape, vtype, integer=False):
    if integer:
        v = rng.integers(-4, 5, shape).astype(np.float64)
        if vtype == "complex64":
            v = v + 1j * rng.integers(-4, 5, shape)
    else:
        v = rng.standard_normal(shape)
        if vtype == "complex64":
            v = v + 1j * rng.standard_normal(shape)
    return storage(v, vtype)


def _dev(arr, vtype=None):
    return to_torch(arr, vtype, DEV)


def _bytes(a):
    return np.ascontiguousarray(a).view(np.uint8)


def _abs_scale(data, indices, indptr, X, n_rows, n_cols, vtype):
    """sum_i |a_ij| |x_i| per output (float64); columns out of range add
    nothing."""
    a = np.abs(widen(data, vtype))
    x = np.abs(widen(X, vtype))
    rows = np.repeat(np.arange(n_rows), np.diff(indptr.astype(np.int64)))
    cols = indices.astype(np.int64)
    ok = (cols >= 0) & (cols < n_cols)
    out = np.zeros((n_cols,) + x.shape[1:])
    np.add.at(out, cols[ok], (a.reshape((-1,) + (1,) * (x.ndim - 1)) * x[rows])[ok])
    return out


@pytest.mark.parametrize("vtype", VTYPES)
@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_transpose_bit_exact(vtype, index_dtype):
    rng = np.random.default_rng(1)
    n_rows, n_cols = 2500, 1800
    indices, indptr, nnz = _matrix(rng, n_rows, n_cols, index_dtype)
    data = _values(rng, nnz, vtype)
    print(f"transpose {vtype} {np.dtype(index_dtype).name} nnz={nnz}", flush=True)
    td, ti, tp = _capi.transpose(_dev(data, vtype), _dev(indices), _dev(indptr), n_rows, n_cols)
    torch.cuda.synchronize()
    wd, wi, wp = orc.csr_transpose(data, indices, indptr, n_rows, n_cols, vtype=vtype)
    np.testing.assert_array_equal(to_numpy(tp), wp)
    np.testing.assert_array_equal(to_numpy(ti), wi)
    np.testing.assert_array_equal(_bytes(to_numpy(td)), _bytes(wd))


def test_transpose_large_and_edges():
    rng = np.random.default_rng(2)
    n = 1 << 20
    indptr = (np.arange(n + 1, dtype=np.int64) * 16).astype(np.int32)
    indices = rng.integers(0, n, n * 16).astype(np.int32)
    data = rng.standard_normal(n * 16).astype(np.float32)
    print(f"transpose large n={n} nnz={n * 16}", flush=True)
    td, ti, tp = _capi.transpose(_dev(data), _dev(indices), _dev(indptr), n, n)
    torch.cuda.synchronize()
    wd, wi, wp = orc.csr_transpose(data, indices, indptr, n, n)
    np.testing.assert_array_equal(to_numpy(tp), wp)
    np.testing.assert_array_equal(to_numpy(ti), wi)
    np.testing.assert_array_equal(to_numpy(td), wd)
    # empty matrix, zero columns, all rows empty
    f = torch.float32
    for n_rows, n_cols in ((0, 7), (5, 0), (6, 9)):
        d = torch.zeros(0, dtype=f, device=DEV)
        i = torch.zeros(0, dtype=torch.int32, device=DEV)
        p = torch.zeros(n_rows + 1, dtype=torch.int32, device=DEV)
        print(f"transpose empty {n_rows}x{n_cols}", flush=True)
        _, _, tp = _capi.transpose(d, i, p, n_rows, n_cols)
        assert tp.tolist() == [0] * (n_cols + 1)


@pytest.mark.parametrize("vtype", VTYPES)
@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_spmv_transpose(vtype, index_dtype):
    rng = np.random.default_rng(3)
    n_rows, n_cols = 3000, 1700
    indices, indptr, nnz = _matrix(rng, n_rows, n_cols, index_dtype)
    # exact case: every partial sum is a small integer, so any order agrees
    data = _values(rng, nnz, vtype, integer=True)
    x = _values(rng, n_rows, vtype, integer=True)
    print(f"spmv_transpose exact {vtype} {np.dtype(index_dtype).name}", flush=True)
    got = _capi.spmv_transpose(_dev(data, vtype), _dev(indices), _dev(indptr), _dev(x, vtype),
                               n_rows, n_cols)
    want = orc.csr_transpose_product(data, indices, indptr, x, n_rows, n_cols, vtype=vtype)
    np.testing.assert_array_equal(_bytes(to_numpy(got)), _bytes(want))
    # rounding case
    data = _values(rng, nnz, vtype)
    x = _values(rng, n_rows, vtype)
    print(f"spmv_transpose tol {vtype} {np.dtype(index_dtype).name}", flush=True)
    got = to_numpy(_capi.spmv_transpose(_dev(data, vtype), _dev(indices), _dev(indptr),
                                        _dev(x, vtype), n_rows, n_cols))
    want = orc.csr_transpose_product(data, indices, indptr, x, n_rows, n_cols, vtype=vtype)
    scale = _abs_scale(data, indices, indptr, x, n_rows, n_cols, vtype)
    err = np.abs(widen(got, vtype) - widen(want, vtype))
    assert np.all(err <= TOL[vtype] * scale + 1e-30), float(np.max(err - TOL[vtype] * scale))


@pytest.mark.parametrize("vtype", VTYPES)
@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_spmv_transpose_wide_output(vtype, index_dtype):
    """1.5 M columns (accumulators of 6 or 12 MB, more than one XCD's L2)
    and columns out of range, which the scatter drops: integer values give
    an exact result in any order of the atomics, random ones stay within
    the tolerance."""
    rng = np.random.default_rng(33)
    n_rows, n_cols = 200_000, 1_500_000
    indices, indptr, nnz = _matrix(rng, n_rows, n_cols, index_dtype)
    indices[rng.random(nnz) < 0.001] = -1
    indices[rng.random(nnz) < 0.001] = n_cols + 3
    data = _values(rng, nnz, vtype, integer=True)
    x = _values(rng, n_rows, vtype, integer=True)
    print(f"spmv_transpose wide exact {vtype} {np.dtype(index_dtype).name}", flush=True)
    got = _capi.spmv_transpose(_dev(data, vtype), _dev(indices), _dev(indptr), _dev(x, vtype),
                               n_rows, n_cols)
    want = orc.csr_transpose_product(data, indices, indptr, x, n_rows, n_cols, vtype=vtype)
    np.testing.assert_array_equal(_bytes(to_numpy(got)), _bytes(want))
    data = _values(rng, nnz, vtype)
    x = _values(rng, n_rows, vtype)
    print(f"spmv_transpose wide tol {vtype} {np.dtype(index_dtype).name}", flush=True)
    got = to_numpy(_capi.spmv_transpose(_dev(data, vtype), _dev(indices), _dev(indptr),
                                        _dev(x, vtype), n_rows, n_cols))
    want = orc.csr_transpose_product(data, indices, indptr, x, n_rows, n_cols, vtype=vtype)
    scale = _abs_scale(data, indices, indptr, x, n_rows, n_cols, vtype)
    err = np.abs(widen(got, vtype) - widen(want, vtype))
    assert np.all(err <= TOL[vtype] * scale + 1e-30), float(np.max(err - TOL[vtype] * scale))


@pytest.mark.parametrize("vtype", VTYPES)
@pytest.mark.parametrize("k", [1, 3, 64, 100])
def test_spmm_transpose_with_padding(vtype, k):
    rng = np.random.default_rng(4 + k)
    n_rows, n_cols = 1200, 900
    indices, indptr, nnz = _matrix(rng, n_rows, n_cols, np.int32)
    data = _values(rng, nnz, vtype, integer=True)
    X = _values(rng, (n_rows, k), vtype, integer=True)
    ldx, ldy = k + 5, k + 3
    Xp = torch.zeros((n_rows, ldx), dtype=_dev(X, vtype).dtype, device=DEV)
    Xp[:, :k] = _dev(X, vtype)
    sentinel = torch.full((n_cols, ldy), 7.0, device=DEV).to(Xp.dtype)
    print(f"spmm_transpose {vtype} k={k}", flush=True)
    _capi.spmm_transpose(_dev(data, vtype), _dev(indices), _dev(indptr), Xp[:, :k], n_rows,
                         n_cols, Y=sentinel, ldy=ldy)
    want = orc.csr_transpose_product(data, indices, indptr, X, n_rows, n_cols, vtype=vtype)
    got = to_numpy(sentinel[:, :k].contiguous())
    np.testing.assert_array_equal(_bytes(got), _bytes(want))
    assert torch.all(sentinel[:, k:] == 7.0)


@pytest.mark.parametrize("vtype", VTYPES)
@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_data_vjp_bit_exact(vtype, index_dtype):
    rng = np.random.default_rng(6)
    n_rows, n_cols = 2000, 1300
    indices, indptr, nnz = _matrix(rng, n_rows, n_cols, index_dtype)
    x = _values(rng, n_cols, vtype)
    cot = _values(rng, n_rows, vtype)
    print(f"data_vjp spmv {vtype} {np.dtype(index_dtype).name}", flush=True)
    got = _capi.spmv_data_vjp(_dev(indices), _dev(indptr), _dev(x, vtype), _dev(cot, vtype),
                              n_rows, n_cols)
    want = orc.csr_data_vjp(indices, indptr, x, cot, n_rows, n_cols, nnz, vtype=vtype)
    np.testing.assert_array_equal(_bytes(to_numpy(got)), _bytes(want))
    for k in (1, 5, 70):
        X = _values(rng, (n_cols, k), vtype)
        C = _values(rng, (n_rows, k), vtype)
        Xd = torch.zeros((n_cols, k + 2), dtype=_dev(X, vtype).dtype, device=DEV)
        Xd[:, :k] = _dev(X, vtype)
        Cd = torch.zeros((n_rows, k + 1), dtype=Xd.dtype, device=DEV)
        Cd[:, :k] = _dev(C, vtype)
        print(f"data_vjp spmm {vtype} k={k}", flush=True)
        got = _capi.spmm_data_vjp(_dev(indices), _dev(indptr), Xd[:, :k], Cd[:, :k], n_rows,
                                  n_cols)
        want = orc.csr_data_vjp(indices, indptr, X, C, n_rows, n_cols, nnz, vtype=vtype)
        np.testing.assert_array_equal(_bytes(to_numpy(got)), _bytes(want))


@pytest.mark.parametrize("vtype", VTYPES)
@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
@pytest.mark.parametrize("bad_cols", [False, True])
def test_data_vjp_through_panel_plan(vtype, index_dtype, bad_cols):
    """The value gradient through a panel plan (x gathered from LDS and
    placed at the tiles' words, the gradient stored in position order):
    equal to the oracle bit for bit, long rows (virtual rows) included.  A
    copy that dropped invalid columns takes the plan-free kernel (zeros
    there)."""
    rng = np.random.default_rng(12)
    n_rows, n_cols = 9000, 200_000
    lengths = rng.integers(0, 40, n_rows)
    lengths[[5, 4000, 8998]] = [3000, 9000, 700]
    indptr = np.zeros(n_rows + 1, np.int64)
    np.cumsum(lengths, out=indptr[1:])
    nnz = int(indptr[-1])
    indices = rng.integers(0, n_cols, nnz)
    if bad_cols:
        indices[rng.random(nnz) < 0.002] = -1
        indices[rng.random(nnz) < 0.002] = n_cols + 5
    indices, indptr = indices.astype(index_dtype), indptr.astype(index_dtype)
    data = _values(rng, nnz, vtype)
    x = _values(rng, n_cols, vtype)
    cot = _values(rng, n_rows, vtype)
    want = orc.csr_data_vjp(indices, indptr, x, cot, n_rows, n_cols, nnz, vtype=vtype)
    d, i, p = _dev(data, vtype), _dev(indices), _dev(indptr)
    for W in (64, 256):
        plan = _capi.Plan(p, n_rows, nnz, W, data=d, indices=i, n_cols=n_cols,
                          slice_mode=_capi.SLICE_PANELS)
        assert plan.info().n_panels > 0
        print(f"data_vjp panels {vtype} {np.dtype(index_dtype).name} W={W} bad={bad_cols}",
              flush=True)
        for _ in range(2):
            got = _capi.spmv_data_vjp(i, p, _dev(x, vtype), _dev(cot, vtype), n_rows, n_cols,
                                      plan=plan)
            np.testing.assert_array_equal(_bytes(to_numpy(got)), _bytes(want))
        plan.close()


@pytest.mark.parametrize("vtype", ["float32", "complex64"])
@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_data_vjp_through_panel_plan_rows_past_bitmap_words(vtype, index_dtype):
    """Rows of 65..256 values and no long row (W = 256): a row's gap word
    lies one to four 64-word bitmap words after its first value, with words
    holding no gap in between, so each value finds its row's gap through
    the next-gap table of its bitmap word.  Empty rows, rows of one value
    and a last row that ends the matrix are mixed in.  Bit-exact against
    the oracle."""
    rng = np.random.default_rng(31)
    n_rows, n_cols = 4000, 150_000
    lengths = rng.integers(65, 256, n_rows)
    lengths[rng.random(n_rows) < 0.05] = 0
    lengths[rng.random(n_rows) < 0.05] = 1
    lengths[-1] = 255
    indptr = np.zeros(n_rows + 1, np.int64)
    np.cumsum(lengths, out=indptr[1:])
    nnz = int(indptr[-1])
    indices = rng.integers(0, n_cols, nnz).astype(index_dtype)
    indptr = indptr.astype(index_dtype)
    data = _values(rng, nnz, vtype)
    x = _values(rng, n_cols, vtype)
    cot = _values(rng, n_rows, vtype)
    want = orc.csr_data_vjp(indices, indptr, x, cot, n_rows, n_cols, nnz, vtype=vtype)
    d, i, p = _dev(data, vtype), _dev(indices), _dev(indptr)
    plan = _capi.Plan(p, n_rows, nnz, 256, data=d, indices=i, n_cols=n_cols,
                      slice_mode=_capi.SLICE_PANELS)
    info = plan.info()
    assert info.n_panels > 0 and info.n_long_rows == 0
    print(f"data_vjp panels wide rows {vtype} {np.dtype(index_dtype).name}", flush=True)
    for _ in range(2):
        got = _capi.spmv_data_vjp(i, p, _dev(x, vtype), _dev(cot, vtype), n_rows, n_cols,
                                  plan=plan)
        np.testing.assert_array_equal(_bytes(to_numpy(got)), _bytes(want))
    plan.close()


@pytest.mark.parametrize("vtype", VTYPES)
def test_deterministic_route_equals_one_worker_reference(vtype):
    # transpose, then the zero-start stored-order SpMM with k = 1: every
    # output summed from zero over its column's values in row order, which
    # is the reference's one-worker transposed product
    rng = np.random.default_rng(8)
    n_rows, n_cols = 2200, 1500
    indices, indptr, nnz = _matrix(rng, n_rows, n_cols, np.int32)
    data = _values(rng, nnz, vtype)
    x = _values(rng, n_rows, vtype)
    print(f"deterministic route {vtype}", flush=True)
    td, ti, tp = _capi.transpose(_dev(data, vtype), _dev(indices), _dev(indptr), n_rows, n_cols)
    y = _capi.spmm(td, ti, tp, _dev(x, vtype).reshape(n_rows, 1), n_cols, n_rows)
    want = orc.csr_transpose_product(data, indices, indptr, x, n_rows, n_cols, vtype=vtype,
                                     n_threads=1)
    np.testing.assert_array_equal(_bytes(to_numpy(y).reshape(-1)), _bytes(want))


def test_adjoint_identity_headline_size():
    n, per_row = 1 << 22, 16
    g = torch.Generator(device=DEV).manual_seed(9)
    indices = torch.randint(0, n, (n * per_row,), device=DEV, dtype=torch.int32, generator=g)
    indptr = torch.arange(0, n * per_row + 1, per_row, device=DEV, dtype=torch.int32)
    data = torch.randn(n * per_row, device=DEV, generator=g)
    x = torch.randn(n, device=DEV, generator=g)
    y = torch.randn(n, device=DEV, generator=g)
    print("adjoint identity n=2^22", flush=True)
    Ax = _capi.spmv(data, indices, indptr, x, n, n)
    Aty = _capi.spmv_transpose(data, indices, indptr, y, n, n)
    absAx = _capi.spmv(data.abs(), indices, indptr, x.abs(), n, n)
    lhs = torch.dot(Ax.double(), y.double()).item()
    rhs = torch.dot(x.double(), Aty.double()).item()
    scale = torch.dot(absAx.double(), y.abs().double()).item()
    assert abs(lhs - rhs) <= 2e-6 * scale, (lhs, rhs, scale)
    # per output: the atomic scatter against the transpose-then-SpMV route
    print("transpose + spmv at n=2^22", flush=True)
    td, ti, tp = _capi.transpose(data, indices, indptr, n, n)
    assert int(tp[-1]) == n * per_row
    det = _capi.spmv(td, ti, tp, y, n, n)
    bound = _capi.spmv(td.abs(), ti, tp, y.abs(), n, n)
    assert torch.all((Aty - det).abs() <= 1e-5 * bound + 1e-30)


def test_adjoint_errors():
    f = torch.float32
    d = torch.ones(1, dtype=f, device=DEV)
    i = torch.zeros(1, dtype=torch.int32, device=DEV)
    p = torch.tensor([0, 1], dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError, match="non-negative"):
        _capi.spmv_transpose(d, i, p, d, -1, 1)
    X = torch.ones(1, 4, device=DEV)
    Y = torch.empty(1, 4, device=DEV)
    L = _capi.lib()
    st = L.msx_csr_spmm_transpose(0, 0, 1, 1, 1, d.data_ptr(), i.data_ptr(), p.data_ptr(), 4,
                                  X.data_ptr(), 2, Y.data_ptr(), 4, _capi._stream())
    assert st == _capi.EINVAL and "leading dimensions" in _capi.last_error()
