"""HIP SpMM parity with the CPU oracle, through the C ABI and the drop-in API.

Each output column is summed from zero in stored order on both sides, so
float32 results must be equal; other dtypes within tol * sum_j |a_ij x_jc|
(1e-5 complex64, 1e-2 float16/bfloat16).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import _capi
from _util import assert_rows_close, storage, to_numpy, to_torch, widen
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

DEV = "cuda"
VTYPES = ["float32", "float16", "bfloat16", "complex64"]


def _values(rng, shape, vtype):
    v = rng.standard_normal(shape)
    if vtype == "complex64":
        v = v + 1j * rng.standard_normal(shape)
    return storage(v, vtype)


def _matrix(rng, n_rows, n_cols, max_len, index_dtype):
    lengths = rng.integers(0, max_len, n_rows)
    lengths[rng.random(n_rows) < 0.1] = 0
    indptr = np.zeros(n_rows + 1, np.int64)
    np.cumsum(lengths, out=indptr[1:])
    nnz = int(indptr[-1])
    return rng.integers(0, n_cols, nnz).astype(index_dtype), indptr.astype(index_dtype), nnz


def _check(data, indices, indptr, X, n_rows, n_cols, vtype, what):
    want = orc.csr_matmul(data, indices, indptr, X, n_rows, vtype=vtype, n_threads=8)
    d = to_torch(data, vtype, DEV)
    i = to_torch(indices, None, DEV)
    p = to_torch(indptr, None, DEV)
    Y = _capi.spmm(d, i, p, to_torch(X, vtype, DEV), n_rows, n_cols)
    torch.cuda.synchronize()
    got = to_numpy(Y)
    if vtype == "float32":
        np.testing.assert_array_equal(got, want, err_msg=what)
    else:
        scale = orc.row_scale(data, indices, indptr, X, n_rows, vtype=vtype)
        assert_rows_close(got, want, scale, vtype, what)
    return got


@pytest.mark.parametrize("vtype", VTYPES)
@pytest.mark.parametrize("k", [1, 2, 3, 7, 8, 16, 32, 33, 64, 128, 256, 300])
def test_widths(vtype, k):
    rng = np.random.default_rng(k)
    indices, indptr, nnz = _matrix(rng, 700, 500, 25, np.int32)
    _check(_values(rng, nnz, vtype), indices, indptr, _values(rng, (500, k), vtype), 700, 500,
           vtype, f"{vtype} k={k}")


@pytest.mark.parametrize("vtype", VTYPES)
def test_int64_and_long_rows(vtype):
    rng = np.random.default_rng(4)
    indices, indptr, nnz = _matrix(rng, 300, 9000, 30, np.int64)
    lengths = np.diff(indptr)
    lengths[[3, 77, 200]] = [5000, 12000, 9000]
    indptr = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    indices = rng.integers(0, 9000, int(indptr[-1])).astype(np.int64)
    _check(_values(rng, indices.size, vtype), indices, indptr, _values(rng, (9000, 16), vtype),
           300, 9000, vtype, f"long {vtype}")


def test_padded_leading_dimensions_and_scalar_path():
    rng = np.random.default_rng(8)
    indices, indptr, nnz = _matrix(rng, 400, 300, 20, np.int32)
    data = _values(rng, nnz, "float32")
    Xfull = _values(rng, (300, 40), "float32")
    want = orc.csr_matmul(data, indices, indptr, np.ascontiguousarray(Xfull[:, :32]), 400)
    d, i, p = (to_torch(a, None, DEV) for a in (data, indices, indptr))
    Xt = to_torch(Xfull, None, DEV)
    # ldx = 40 (multiple of 4): vector path on a padded X; ldy = 36
    Yb = torch.full((400, 36), 7.0, device=DEV)
    _capi.spmm(d, i, p, Xt[:, :32], 400, 300, Y=Yb, ldx=40, ldy=36)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(Yb[:, :32].cpu().numpy(), want)
    assert torch.all(Yb[:, 32:] == 7.0)  # padding untouched
    # ldx = 39: scalar path
    X39 = to_torch(np.ascontiguousarray(Xfull[:, :39]), None, DEV)
    Y = _capi.spmm(d, i, p, X39[:, :32], 400, 300, ldx=39, ldy=32)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(Y.cpu().numpy(), want)


@pytest.mark.parametrize("vtype", VTYPES)
def test_two_line_rows_padded_and_out_of_range(vtype):
    """X rows of exactly two 128-byte lines take the line-tiled kernel: padded
    leading dimensions, a row count that is not a multiple of the row groups,
    and indices outside [0, n_cols), which contribute nothing."""
    k = 256 // storage(np.zeros(1), vtype).itemsize
    rng = np.random.default_rng(11)
    n_rows, n_cols = 1001, 600
    indices, indptr, nnz = _matrix(rng, n_rows, n_cols, 40, np.int32)
    bad = rng.random(nnz) < 0.05
    indices = indices.copy()
    indices[bad] = np.where(rng.random(int(bad.sum())) < 0.5, -3, n_cols + 7)
    data = _values(rng, nnz, vtype)
    Xfull = _values(rng, (n_cols, k + 8), vtype)
    X = np.ascontiguousarray(Xfull[:, :k])
    keep = ~bad
    row_of = np.repeat(np.arange(n_rows), np.diff(indptr))
    kept_ptr = np.concatenate([[0], np.cumsum(np.bincount(row_of[keep], minlength=n_rows))])
    kept_ptr = kept_ptr.astype(np.int32)
    want = orc.csr_matmul(data[keep], indices[keep], kept_ptr, X, n_rows, vtype=vtype)
    d, i, p = (to_torch(a, vtype if a is data else None, DEV) for a in (data, indices, indptr))
    Xt = to_torch(Xfull, vtype, DEV)
    Yb = torch.zeros((n_rows, k + 8), dtype=Xt.dtype, device=DEV)
    Yb[:, k:] = 5
    _capi.spmm(d, i, p, Xt[:, :k], n_rows, n_cols, Y=Yb, ldx=k + 8, ldy=k + 8)
    torch.cuda.synchronize()
    assert torch.all(Yb[:, k:] == 5)  # padding untouched
    got = to_numpy(Yb)
    if vtype == "float32":
        np.testing.assert_array_equal(got[:, :k], want)
    else:
        scale = orc.row_scale(data[keep], indices[keep], kept_ptr, X, n_rows, vtype=vtype)
        assert_rows_close(np.ascontiguousarray(got[:, :k]), want, scale, vtype, vtype)


def test_golden_widths_and_batched_api(gpu):
    from pathlib import Path

    ms = gpu
    z = np.load(Path(__file__).parent / "golden" / "scipy_cases.npz")
    for k in (1, 2, 4, 8, 16, 32):
        pre = f"widths{k}"
        shape = tuple(int(v) for v in z[f"{pre}.shape"])
        A = ms.csr_array((z[f"{pre}.data"], z[f"{pre}.indices"], z[f"{pre}.indptr"]), shape=shape)
        Y = (A @ torch.from_numpy(z[f"{pre}.X"]).to(DEV)).cpu().numpy()
        np.testing.assert_allclose(Y, z[f"{pre}.scipy"], rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(Y, z[f"{pre}.dense64"], rtol=1e-5, atol=1e-5)
    # batched RHS (reference tests/test_numerical_correctness.py:76-80)
    shape = tuple(int(v) for v in z["numcorr.shape"])
    A = ms.csr_array((z["numcorr.data"], z["numcorr.indices"], z["numcorr.indptr"]), shape=shape)
    out = (A @ torch.from_numpy(z["numcorr.B"]).to(DEV)).cpu().numpy()
    np.testing.assert_allclose(out, z["numcorr.dense64_B"], rtol=1e-5, atol=1e-5)
    # complex (reference tests/test_numerical_correctness.py:83-113)
    shape = tuple(int(v) for v in z["complex.shape"])
    C = ms.csr_array((z["complex.data"], z["complex.indices"], z["complex.indptr"]), shape=shape)
    np.testing.assert_allclose((C @ torch.from_numpy(z["complex.X"]).to(DEV)).cpu().numpy(),
                               z["complex.dense128_X"], rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose((C @ torch.from_numpy(z["complex.x"]).to(DEV)).cpu().numpy(),
                               z["complex.dense128_x"], rtol=1e-5, atol=1e-5)


def test_poisson_spmm_k64_full_size():
    """The SpMM benchmark matrix at full size: column c equals SpMV of X[:, c]
    (checked on 4 columns) and the whole product equals the oracle."""
    from mlx_sparse import synthetic

    m = synthetic.poisson_3d(128)
    X = synthetic.normal(m.shape[1], seed=2, k=64)
    got = _check(m.data, m.indices, m.indptr, X, m.shape[0], m.shape[1], "float32", "poisson k=64")
    d, i, p = (to_torch(a, None, DEV) for a in (m.data, m.indices, m.indptr))
    plan = _capi.Plan(p, m.shape[0], m.nnz)  # short blocks sum rows in stored order
    for c in (0, 17, 40, 63):
        y = _capi.spmv(d, i, p, to_torch(np.ascontiguousarray(X[:, c]), None, DEV), m.shape[0],
                       m.shape[1], plan=plan)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(to_numpy(y), got[:, c])


# -- column windows of bound plans (banded matrices) ---------------------------------


def _banded(n, half_band, seed, vtype, index_dtype=np.int32):
    from mlx_sparse import synthetic

    m = synthetic.banded(n, half_band, 0.65, 10.0, seed=seed, index_dtype=index_dtype)
    rng = np.random.default_rng(seed)
    return m, _values(rng, m.nnz, vtype)


@pytest.mark.parametrize("vtype", VTYPES)
@pytest.mark.parametrize("k", [4, 8, 16, 32, 48, 64, 128, 256])
def test_window_spmm_matches_oracle_and_plan_free(vtype, k):
    """A bound plan of a banded matrix records each 32-row tile's column
    window; the SpMM then gathers X from LDS.  Same sums as without the plan
    (bit for bit) and as the oracle (float32 bit for bit) - except float16 /
    bfloat16 with k a multiple of 16, which run on the matrix cores (float32
    accumulation in the MFMA's order): within the 16-bit tolerance of both."""
    n, hb = 3001, 12  # n not a multiple of the 32-row tile
    m, data = _banded(n, hb, seed=k, vtype=vtype)
    rng = np.random.default_rng(100 + k)
    X = _values(rng, (n, k), vtype)
    d, i, p = to_torch(data, vtype, DEV), to_torch(m.indices, None, DEV), to_torch(m.indptr, None, DEV)
    plan = _capi.Plan(p, n, m.nnz, data=d, indices=i, n_cols=n)
    w = plan.info().window_rows
    assert 32 <= w <= 32 + 2 * hb, w  # a full tile plus the band on each side
    Xt = to_torch(X, vtype, DEV)
    got = _capi.spmm(d, i, p, Xt, n, n, plan=plan)
    ref = _capi.spmm(d, i, p, Xt, n, n)
    torch.cuda.synchronize()
    want = orc.csr_matmul(data, m.indices, m.indptr, X, n, vtype=vtype, n_threads=8)
    scale = orc.row_scale(data, m.indices, m.indptr, X, n, vtype=vtype)
    mfma = vtype in ("float16", "bfloat16") and k in (16, 32, 64, 128, 256)
    if mfma:
        assert_rows_close(to_numpy(got), to_numpy(ref), scale, vtype, f"window mfma {vtype} k={k}")
    else:
        np.testing.assert_array_equal(to_numpy(got), to_numpy(ref))
    if vtype == "float32":
        np.testing.assert_array_equal(to_numpy(got), want)
    else:
        assert_rows_close(to_numpy(got), want, scale, vtype, f"window {vtype} k={k}")
    plan.close()


@pytest.mark.parametrize("vtype", ["float16", "bfloat16"])
def test_window_mfma_tiles_that_keep_stored_order(vtype):
    """Tiles the matrix cores cannot take - a repeated (row, column) pair, a
    column moved outside the tile's recorded window - are summed in stored
    order from global memory, equal to the oracle bit for bit; the other
    tiles stay within the 16-bit tolerance; out-of-range columns add
    nothing."""
    n, k = 2000, 64
    m, data = _banded(n, 6, seed=9, vtype=vtype)
    rng = np.random.default_rng(10)
    X = _values(rng, (n, k), vtype)
    idx = m.indices.copy()
    d, i, p = to_torch(data, vtype, DEV), to_torch(idx, None, DEV), to_torch(m.indptr, None, DEV)
    plan = _capi.Plan(p, n, m.nnz, data=d, indices=i, n_cols=n)
    assert plan.info().window_rows > 0
    ip = m.indptr.astype(np.int64)
    r_dup, r_far = 100, 700  # tiles 3 and 21
    idx[ip[r_dup] + 1] = idx[ip[r_dup]]             # repeated column in one row
    idx[ip[r_far]] = (idx[ip[r_far]] + n // 2) % n   # far outside its tile's window
    idx[ip[1500]] = n + 3                            # out of range: adds nothing
    i.copy_(to_torch(idx, None, DEV))
    got = to_numpy(_capi.spmm(d, i, p, to_torch(X, vtype, DEV), n, n, plan=plan))
    keep = (idx >= 0) & (idx < n)
    rows = np.repeat(np.arange(n), np.diff(ip))
    kept_indptr = np.concatenate([[0], np.cumsum(np.bincount(rows[keep], minlength=n))])
    kidx, kptr = idx[keep].astype(np.int64), kept_indptr.astype(np.int64)
    want = orc.csr_matmul(data[keep], kidx, kptr, X, n, vtype=vtype, n_threads=8)
    for r in (r_dup, r_far):
        t = r // 32
        np.testing.assert_array_equal(got[32 * t:32 * t + 32], want[32 * t:32 * t + 32],
                                      err_msg=f"stored-order tile {t}")
    scale = orc.row_scale(data[keep], kidx, kptr, X, n, vtype=vtype)
    assert_rows_close(got, want, scale, vtype, f"window mfma {vtype} edited")
    plan.close()


@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_window_mfma_repeated_columns_at_every_lane_boundary(index_dtype):
    """Eight lanes take a row's entries, four per lane and step (entry e on
    lane e % 8, step e // 32): a repeated column is caught whether the pair
    sits on neighbouring lanes (0, 1), across the group's wrap (7, 8) or
    across two steps (31, 32); its tile keeps the stored-order sum, equal to
    the oracle bit for bit."""
    vtype, n, k = "float16", 4000, 64
    m, data = _banded(n, 24, seed=31, vtype=vtype, index_dtype=index_dtype)
    rng = np.random.default_rng(32)
    X = _values(rng, (n, k), vtype)
    ip = m.indptr.astype(np.int64)
    idx = m.indices.copy()
    rows = {}
    lengths = np.diff(ip)
    for r0, (a, b) in zip((330, 1650, 2990), ((0, 1), (7, 8), (31, 32))):
        r = r0 + int(np.argmax(lengths[r0:] > b))  # the first row from r0 long enough
        assert lengths[r] > b, (r, lengths[r])
        idx[ip[r] + b] = idx[ip[r] + a]
        rows[r] = (a, b)
    d, i, p = to_torch(data, vtype, DEV), to_torch(idx, None, DEV), to_torch(m.indptr, None, DEV)
    plan = _capi.Plan(p, n, m.nnz, data=d, indices=i, n_cols=n)
    assert plan.info().window_rows > 0
    got = to_numpy(_capi.spmm(d, i, p, to_torch(X, vtype, DEV), n, n, plan=plan))
    torch.cuda.synchronize()
    want = orc.csr_matmul(data, idx.astype(np.int64), ip, X, n, vtype=vtype, n_threads=8)
    for r in rows:
        t = r // 32
        np.testing.assert_array_equal(got[32 * t:32 * t + 32], want[32 * t:32 * t + 32],
                                      err_msg=f"stored-order tile {t}, pair {rows[r]}")
    scale = orc.row_scale(data, idx.astype(np.int64), ip, X, n, vtype=vtype)
    assert_rows_close(got, want, scale, vtype, "window mfma repeated columns")
    plan.close()


@pytest.mark.parametrize("vtype", ["float16", "bfloat16"])
def test_window_mfma_nonfinite_x_and_unsorted_rows(vtype):
    """An infinite or NaN X value inside a tile's window would reach every
    row of the tile through the zeros of its dense block (0 x inf), so that
    tile keeps the stored-order sum: equal to the oracle bit for bit, finite
    in the rows that do not read it.  A row whose columns decrease (no
    repeated pair) stays on the matrix cores, within the 16-bit tolerance."""
    n, k = 3000, 64
    m, data = _banded(n, 8, seed=21, vtype=vtype)
    rng = np.random.default_rng(22)
    X = _values(rng, (n, k), vtype).copy()
    ip = m.indptr.astype(np.int64)
    idx = m.indices.copy()
    r_rev = 1000  # tile 31: its row's columns reversed
    idx[ip[r_rev]:ip[r_rev + 1]] = idx[ip[r_rev]:ip[r_rev + 1]][::-1].copy()
    c_inf, c_nan = 455, 2001  # tiles 14 and 62
    X[c_inf, 3] = storage(np.array([np.inf]), vtype)[0]
    X[c_nan, 40] = storage(np.array([np.nan]), vtype)[0]
    d, i, p = to_torch(data, vtype, DEV), to_torch(idx, None, DEV), to_torch(m.indptr, None, DEV)
    plan = _capi.Plan(p, n, m.nnz, data=d, indices=i, n_cols=n)
    assert plan.info().window_rows > 0
    got = to_numpy(_capi.spmm(d, i, p, to_torch(X, vtype, DEV), n, n, plan=plan))
    torch.cuda.synchronize()
    want = orc.csr_matmul(data, idx.astype(np.int64), ip, X, n, vtype=vtype, n_threads=8)
    rows = np.repeat(np.arange(n), np.diff(ip))
    tiles_of = rows // 32
    lo = np.full(-(-n // 32), n, np.int64)
    hi = np.full(-(-n // 32), -1, np.int64)
    np.minimum.at(lo, tiles_of, idx.astype(np.int64))
    np.maximum.at(hi, tiles_of, idx.astype(np.int64))
    for c, expect in ((c_inf, {13, 14}), (c_nan, {62})):
        # every tile whose window [lowest, highest column] holds X row c:
        # at half-bandwidth 8 also the tile before c // 32 when c sits low
        tiles = set(np.flatnonzero((lo <= c) & (c <= hi)).tolist())
        assert expect <= tiles, (c, sorted(tiles))
        for t in sorted(tiles):
            g, w = widen(got[32 * t:32 * t + 32], vtype), widen(want[32 * t:32 * t + 32], vtype)
            assert np.array_equal(g, w, equal_nan=True), f"stored-order tile {t} (X row {c})"
            readers = np.unique(rows[idx == c])
            others = np.setdiff1d(np.arange(32 * t, min(32 * t + 32, n)), readers)
            assert len(others) > 0 and np.isfinite(widen(got[others], vtype)).all(), \
                f"tile {t}: rows that do not read X row {c} must stay finite"
    Xf = np.where(np.isfinite(widen(X, vtype)), X, storage(np.zeros(1), vtype)[0])
    scale = orc.row_scale(data, idx.astype(np.int64), ip, Xf, n, vtype=vtype)
    # every entry: within tolerance, or the same non-finite value as the oracle
    assert_rows_close(got, want, scale, vtype, f"window mfma {vtype} non-finite")
    plan.close()


def test_window_spmm_columns_outside_the_recorded_window():
    """Columns moved after the plan was built (same buffers) and columns out
    of range: values outside a tile's recorded window are read from X
    directly, so the product still equals the oracle."""
    n, k = 2000, 32
    m, data = _banded(n, 6, seed=3, vtype="float32", index_dtype=np.int64)
    rng = np.random.default_rng(5)
    X = _values(rng, (n, k), "float32")
    d, i, p = to_torch(data, "float32", DEV), to_torch(m.indices, None, DEV), to_torch(m.indptr, None, DEV)
    plan = _capi.Plan(p, n, m.nnz, data=d, indices=i, n_cols=n)
    assert plan.info().window_rows > 0
    moved = m.indices.copy()
    moved[::97] = (moved[::97] + n // 2) % n  # far outside each tile's window
    moved[5] = n + 7                          # out of range: adds nothing
    i.copy_(to_torch(moved, None, DEV))
    got = _capi.spmm(d, i, p, to_torch(X, "float32", DEV), n, n, plan=plan)
    torch.cuda.synchronize()
    # the GPU skips the out-of-range entry (the reference would read past X):
    # the oracle gets the matrix without it
    keep = (moved >= 0) & (moved < n)
    rows = np.repeat(np.arange(n), np.diff(m.indptr))
    kept_indptr = np.concatenate([[0], np.cumsum(np.bincount(rows[keep], minlength=n))])
    want = orc.csr_matmul(data[keep], moved[keep], kept_indptr.astype(np.int64), X, n,
                          vtype="float32", n_threads=8)
    np.testing.assert_array_equal(to_numpy(got), want)
    plan.close()


def test_window_tile_too_full_to_scan():
    """A tile holding more values than LDS could ever stage (one row of
    20,000 values) is not scanned: the other tiles keep their narrow windows,
    the window kernel is off for the matrix, and the product is unchanged."""
    n, hb, k = 30001, 6, 32
    rng = np.random.default_rng(4)
    rows = [np.arange(max(0, r - hb), min(n, r + hb + 1)) for r in range(n)]
    rows[100] = np.sort(rng.choice(n, 20000, replace=False))
    indptr = np.concatenate([[0], np.cumsum([r.size for r in rows])]).astype(np.int32)
    indices = np.concatenate(rows).astype(np.int32)
    data = _values(rng, indices.size, "float32")
    d, i, p = to_torch(data, "float32", DEV), to_torch(indices, None, DEV), to_torch(indptr, None, DEV)
    plan = _capi.Plan(p, n, indices.size, data=d, indices=i, n_cols=n)
    assert 0 < plan.info().window_rows <= 32 + 2 * hb
    X = _values(rng, (n, k), "float32")
    Xt = to_torch(X, "float32", DEV)
    got = _capi.spmm(d, i, p, Xt, n, n, plan=plan)
    ref = _capi.spmm(d, i, p, Xt, n, n)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_numpy(got), to_numpy(ref))
    np.testing.assert_array_equal(
        to_numpy(got), orc.csr_matmul(data, indices, indptr, X, n, vtype="float32", n_threads=8))
    plan.close()


def test_window_not_used_when_too_wide():
    """A random matrix's tiles span all columns: the window does not fit LDS
    and the SpMM keeps the global-gather kernels (same result either way)."""
    rng = np.random.default_rng(11)
    indices, indptr, nnz = _matrix(rng, 4000, 20000, 20, np.int32)
    data = _values(rng, nnz, "float32")
    d, i, p = to_torch(data, "float32", DEV), to_torch(indices, None, DEV), to_torch(indptr, None, DEV)
    plan = _capi.Plan(p, 4000, nnz, data=d, indices=i, n_cols=20000)
    assert plan.info().window_rows > 10000
    X = _values(rng, (20000, 64), "float32")
    got = _capi.spmm(d, i, p, to_torch(X, "float32", DEV), 4000, 20000, plan=plan)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(
        to_numpy(got), orc.csr_matmul(data, indices, indptr, X, 4000, vtype="float32", n_threads=8))
    plan.close()
