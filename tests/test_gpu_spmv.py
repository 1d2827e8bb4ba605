"""HIP SpMV parity with the CPU oracle, through the C ABI.

Bar: index work (the row-block plan) bit-exact against oracle/plan_oracle.py;
values within |gpu - oracle| <= tol * sum_j |a_ij x_j| per row with tol =
1e-5 (float32, complex64) or 1e-2 (float16, bfloat16).  float32 rows that the
kernels sum in stored order (short blocks with mean row length <= 32, and
the plan-free kernel at one lane per row) are also checked for equality.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import _capi
from _util import TORCH, assert_rows_close, storage, to_numpy, to_torch
from oracle import oracle as orc
from oracle import plan_oracle

pytestmark = pytest.mark.gpu

DEV = "cuda"
VTYPES = ["float32", "float16", "bfloat16", "complex64"]


def _upload(data, indices, indptr, vtype):
    return (to_torch(data, vtype, DEV), to_torch(indices, None, DEV), to_torch(indptr, None, DEV))


def _values(rng, n, vtype):
    v = rng.standard_normal(n)
    if vtype == "complex64":
        v = v + 1j * rng.standard_normal(n)
    return storage(v, vtype)


def _random_csr(rng, n_rows, n_cols, lengths, index_dtype):
    indptr = np.zeros(n_rows + 1, np.int64)
    np.cumsum(lengths, out=indptr[1:])
    nnz = int(indptr[-1])
    indices = rng.integers(0, n_cols, nnz)
    return indices.astype(index_dtype), indptr.astype(index_dtype), nnz


# Rows this long may differ from the oracle by more than the tolerance only
# where the GPU sum is the more accurate one: the oracle's stored-order
# float32 sum has a typical relative error 2^-24 * sqrt(n / 3), which passes
# 1e-5 near n = 10^5 (the power-law matrix holds rows up to 200,000 values).
LONG_ROW_EXEMPT = 10_000


def _check_spmv(data, indices, indptr, x, n_rows, n_cols, vtype, plan_w=0, what=""):
    want = orc.csr_matvec(data, indices, indptr, x, n_rows, vtype=vtype, n_threads=8)
    scale = orc.row_scale(data, indices, indptr, x, n_rows, vtype=vtype)
    exact = orc.row_exact(data, indices, indptr, x, n_rows, vtype=vtype)
    lengths = np.diff(np.asarray(indptr, dtype=np.int64))
    d, i, p = _upload(data, indices, indptr, vtype)
    xt = to_torch(x, vtype, DEV)
    out = {}
    plan = _capi.Plan(p, n_rows, int(data.shape[0]), plan_w) if plan_w is not None else None
    for label, pl in (("plan", plan), ("planfree", None)):
        y = _capi.spmv(d, i, p, xt, n_rows, n_cols, plan=pl)
        torch.cuda.synchronize()
        got = to_numpy(y)
        rep = assert_rows_close(got, want, scale, vtype, f"{what} {label}", exact=exact,
                                lengths=lengths, min_len_exempt=LONG_ROW_EXEMPT)
        if rep["exempt_rows"]:
            print(f"{what} {label}: {rep}")
        out[label] = got
    if plan is not None:
        plan.close()
    return out, want


# -- reference KATs through the drop-in API on the GPU ---------------------------

def test_kat_through_api(gpu):
    ms = gpu
    A = ms.csr_array((np.array([2.0, -1.0, 4.0, 5.0], np.float32), np.array([0, 2, 1, 3], np.int32),
                      np.array([0, 2, 2, 4], np.int32)), shape=(3, 4))
    assert A.data.device.type == "cuda"
    y = A @ np.array([3.0, 10.0, 7.0, -2.0], np.float32)
    assert y.device.type == "cuda"
    np.testing.assert_array_equal(y.cpu().numpy(), [-1.0, 0.0, 30.0])
    # non-contiguous operands (reference tests/test_csr_matvec.py:318-333)
    data = torch.tensor([99.0, 2.0, 99.0, -1.0, 99.0, 4.0, 99.0, 5.0], device=DEV)[1::2]
    idx = torch.tensor([9, 0, 9, 2, 9, 1, 9, 3], dtype=torch.int32, device=DEV)[1::2]
    x = torch.tensor([99.0, 3.0, 99.0, 10.0, 99.0, 7.0, 99.0, -2.0], device=DEV)[1::2]
    B = ms.csr_array((data, idx, torch.tensor([0, 2, 2, 4], dtype=torch.int32)), shape=(3, 4))
    np.testing.assert_array_equal((B @ x).cpu().numpy(), [-1.0, 0.0, 30.0])
    # bfloat16 returns bfloat16 (reference tests/test_dtypes.py:64-77)
    C = ms.csr_array((torch.tensor([2.0, -1.0], dtype=torch.bfloat16), torch.tensor([0, 1], dtype=torch.int32),
                      torch.tensor([0, 2], dtype=torch.int32)), shape=(1, 2))
    yb = C @ torch.tensor([3.0, 7.0], dtype=torch.bfloat16)
    assert yb.dtype == torch.bfloat16 and yb.float().item() == -1.0


def test_errors_through_api(gpu):
    ms = gpu
    A = ms.csr_array((np.ones(1, np.float32), np.zeros(1, np.int32), np.array([0, 1], np.int32)),
                     shape=(1, 2))
    with pytest.raises(ValueError, match="n_cols"):
        A @ torch.ones(1, device=DEV)
    with pytest.raises(TypeError, match="dtype must be one"):
        A @ torch.ones(2, dtype=torch.int32, device=DEV)
    with pytest.raises(TypeError, match="same dtype"):
        A @ torch.ones(2, dtype=torch.float16, device=DEV)


# -- golden fixtures -------------------------------------------------------------

@pytest.mark.parametrize("name", ["well1033", "illc1033", "bcsstk03"])
def test_suitesparse_fixtures(name):
    from pathlib import Path

    z = np.load(Path(__file__).parent / "golden" / f"suitesparse_{name}.npz")
    shape = tuple(int(v) for v in z["shape"])
    out, want = _check_spmv(z["data"], z["indices"], z["indptr"], z["x"], shape[0], shape[1],
                            "float32", what=name)
    np.testing.assert_array_equal(want, z["scipy_x"])
    np.testing.assert_array_equal(out["plan"], want)  # short rows: stored-order sums


# -- dtype x index type sweep with ragged and empty rows ------------------------

@pytest.mark.parametrize("vtype", VTYPES)
@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_random_ragged(vtype, index_dtype):
    rng = np.random.default_rng(100 + VTYPES.index(vtype))
    n_rows, n_cols = 5000, 3000
    lengths = rng.integers(0, 30, n_rows)
    lengths[rng.random(n_rows) < 0.1] = 0
    indices, indptr, nnz = _random_csr(rng, n_rows, n_cols, lengths, index_dtype)
    out, want = _check_spmv(_values(rng, nnz, vtype), indices, indptr, _values(rng, n_cols, vtype),
                            n_rows, n_cols, vtype, what=f"{vtype}/{index_dtype.__name__}")
    if vtype == "float32":
        np.testing.assert_array_equal(out["plan"], want)


@pytest.mark.parametrize("vtype", VTYPES)
def test_long_rows_and_fixup(vtype):
    # lengths straddling W=256 (short/long), C=4096 (one chunk / several)
    rng = np.random.default_rng(7)
    special = [0, 1, 4, 5, 255, 256, 257, 1000, 4095, 4096, 4097, 8192, 12289, 60000]
    lengths = np.concatenate([rng.integers(0, 20, 300), special, rng.integers(0, 3, 500), special[::-1]])
    rng.shuffle(lengths)
    n_rows, n_cols = lengths.size, 70000
    indices, indptr, nnz = _random_csr(rng, n_rows, n_cols, lengths, np.int32)
    _check_spmv(_values(rng, nnz, vtype), indices, indptr, _values(rng, n_cols, vtype), n_rows,
                n_cols, vtype, plan_w=256, what=f"long/{vtype}")


@pytest.mark.parametrize("vtype", VTYPES)
def test_long_rows_sliced_by_column(vtype):
    """A bound plan with x of 4 MB or more cuts long rows with sorted columns
    at the 8 XCD column slices (pieces of at most 1020 values, each slice's
    pieces on its own XCD); a long row with unsorted columns keeps the
    chunked long-row kernel.  Both match the oracle; an out-of-range column
    at the end of a sorted long row adds nothing."""
    rng = np.random.default_rng(31)
    n_rows, n_cols = 3000, 2_200_000
    lengths = rng.integers(0, 20, n_rows)
    special = {17: 300, 400: 1021, 401: 1020, 1200: 5000, 2000: 40000, 2999: 200000, 5: 257}
    for r, L in special.items():
        lengths[r] = L
    cols = []
    for L in lengths:
        c = np.unique(rng.integers(0, n_cols, int(L * 1.2) + 8))
        cols.append(np.sort(rng.permutation(c)[:L]))
    cols[1200][-1] = n_cols + 5  # out of range, still sorted
    indptr = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    indices = np.concatenate(cols).astype(np.int32)
    nnz = int(indptr[-1])
    data = _values(rng, nnz, vtype)
    x = _values(rng, n_cols, vtype)
    keep = indices < n_cols
    rows = np.repeat(np.arange(n_rows), lengths)
    k_indptr = np.concatenate([[0], np.cumsum(np.bincount(rows[keep], minlength=n_rows))]).astype(np.int32)
    want = orc.csr_matvec(data[keep], indices[keep], k_indptr, x, n_rows, vtype=vtype, n_threads=8)
    scale = orc.row_scale(data[keep], indices[keep], k_indptr, x, n_rows, vtype=vtype)
    exact = orc.row_exact(data[keep], indices[keep], k_indptr, x, n_rows, vtype=vtype)
    xt = to_torch(x, vtype, DEV)
    p = to_torch(indptr, None, DEV)
    sizes = []
    for label in ("sorted", "unsorted"):
        if label == "unsorted":  # one long row loses its order: same sums, other kernel
            a, b = int(indptr[2000]), int(indptr[2000]) + 1
            indices[[a, b]] = indices[[b, a]]
            data[[a, b]] = data[[b, a]]
        d, i = to_torch(data, vtype, DEV), to_torch(indices, None, DEV)
        plan = _capi.Plan(p, n_rows, nnz, data=d, indices=i, n_cols=n_cols,
                          slice_mode=_capi.SLICE_OFF)
        sizes.append(plan.info().plan_bytes)
        y = _capi.spmv(d, i, p, xt, n_rows, n_cols, plan=plan)
        torch.cuda.synchronize()
        assert_rows_close(to_numpy(y), want, scale, vtype, f"{label} long rows", exact=exact,
                          lengths=lengths, min_len_exempt=LONG_ROW_EXEMPT)
        plan.close()
    assert sizes[0] > sizes[1]  # only the sorted plan holds the slice pieces


@pytest.mark.parametrize("W", [64, 128, 256, 512, 1024])
def test_plan_bins_bit_exact(W):
    rng = np.random.default_rng(W)
    lengths = rng.integers(0, 50, 20000)
    big = rng.random(lengths.size) < 0.01
    lengths[big] = rng.integers(W + 1, 20 * W, big.sum())
    lengths[5000:6500] = 0  # a long run of empty rows
    for index_dtype in (np.int32, np.int64):
        indptr = np.zeros(lengths.size + 1, np.int64)
        np.cumsum(lengths, out=indptr[1:])
        p = torch.from_numpy(indptr.astype(index_dtype)).to(DEV)
        plan = _capi.Plan(p, lengths.size, int(indptr[-1]), W)
        got = plan.export()
        want = plan_oracle.plan(indptr, W=W)
        for g, w, name in zip(got, want, ("blocks", "long_rows", "chunk_begin")):
            np.testing.assert_array_equal(g, w, err_msg=name)
        info = plan.info()
        assert info.n_bounds == want[0].size - 1 and info.n_long_rows == want[1].size
        assert info.n_blocks == info.n_bounds - info.n_long_rows
        plan.close()


def test_default_block_nnz_follows_mean_row_length():
    # W = 0 asks for the default: 512 when rows average 20 values or more
    for per_row, want_w in ((19, 256), (20, 512), (0, 256)):
        indptr = np.arange(1001, dtype=np.int64) * per_row
        p = torch.from_numpy(indptr.astype(np.int32)).to(DEV)
        plan = _capi.Plan(p, 1000, int(indptr[-1]))
        assert plan.info().block_nnz == want_w
        np.testing.assert_array_equal(plan.export()[0], plan_oracle.plan(indptr, W=want_w)[0])
        plan.close()
    # a bound complex64 plan keeps 256 (its wide blocks would halve occupancy)
    idx = torch.zeros(20000, dtype=torch.int32, device=DEV)
    p = torch.arange(0, 20001, 20, dtype=torch.int32, device=DEV)
    for dtype, want_w in ((torch.complex64, 256), (torch.float32, 512), (torch.bfloat16, 512)):
        plan = _capi.Plan(p, 1000, 20000, data=torch.zeros(20000, dtype=dtype, device=DEV),
                          indices=idx, n_cols=4, slice_mode=_capi.SLICE_OFF)
        assert plan.info().block_nnz == want_w, dtype
        plan.close()


def test_empty_and_degenerate():
    for n_rows, n_cols, lengths in [(0, 5, []), (4, 0, [0, 0, 0, 0]), (3, 7, [0, 0, 0]),
                                    (1, 1, [1]), (2, 3, [3, 0])]:
        lengths = np.asarray(lengths, np.int64)
        rng = np.random.default_rng(0)
        indices, indptr, nnz = _random_csr(rng, n_rows, max(n_cols, 1), lengths, np.int32)
        data = _values(rng, nnz, "float32")
        x = _values(rng, n_cols, "float32")
        d, i, p = _upload(data, indices, indptr, "float32")
        y = _capi.spmv(d, i, p, to_torch(x, None, DEV), n_rows, n_cols,
                       plan=_capi.Plan(p, n_rows, nnz))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(to_numpy(y), orc.csr_matvec(data, indices, indptr, x, n_rows))


def test_out_of_range_columns_add_nothing():
    # malformed input: columns outside [0, n_cols) must not be read
    data = np.ones(6, np.float32)
    indices = np.array([0, -1, 5, 1, 1 << 30, 2], np.int32)
    indptr = np.array([0, 3, 6], np.int32)
    x = np.array([1.0, 2.0, 4.0], np.float32)
    d, i, p = _upload(data, indices, indptr, "float32")
    sliced = _capi.Plan(p, 2, 6, data=d, indices=i, n_cols=3, slice_mode=_capi.SLICE_ON)
    assert sliced.info().n_slices == 8
    panels = _capi.Plan(p, 2, 6, data=d, indices=i, n_cols=3, slice_mode=_capi.SLICE_PANELS)
    assert panels.info().n_panels == 1 and panels.info().panel_values == 4  # 3 values + 1 pad
    for plan in (_capi.Plan(p, 2, 6), None, sliced, panels):
        y = _capi.spmv(d, i, p, to_torch(x, None, DEV), 2, 3, plan=plan)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(to_numpy(y), [1.0, 6.0])


def test_misaligned_buffers_use_plan_free_path():
    rng = np.random.default_rng(3)
    lengths = rng.integers(0, 40, 2000)
    indices, indptr, nnz = _random_csr(rng, 2000, 2000, lengths, np.int32)
    data = _values(rng, nnz + 1, "float32")
    x = _values(rng, 2000, "float32")
    dd = to_torch(data, None, DEV)[1:]  # 4-byte offset: not 16-byte aligned
    ii = to_torch(np.concatenate([[0], indices]).astype(np.int32), None, DEV)[1:]
    p = to_torch(indptr, None, DEV)
    plan = _capi.Plan(p, 2000, nnz)
    y = _capi.spmv(dd, ii, p, to_torch(x, None, DEV), 2000, 2000, plan=plan)
    torch.cuda.synchronize()
    want = orc.csr_matvec(data[1:], indices, indptr, x, 2000)
    assert_rows_close(to_numpy(y), want, orc.row_scale(data[1:], indices, indptr, x, 2000),
                      "float32", "misaligned")


@pytest.mark.parametrize("vtype", ["float16", "bfloat16", "float32"])
def test_x_gathers_at_any_alignment(vtype):
    """The short-block kernel reads 16-bit x elements as the dword that holds
    them when x is dword-aligned, and with plain element loads otherwise (x at
    a 2-byte offset).  n_cols is odd and the last column is used, so the last
    element sits in the low half of a dword whose high half is past x."""
    rng = np.random.default_rng(17)
    n_rows, n_cols = 3000, 2001
    lengths = rng.integers(0, 40, n_rows)
    indices, indptr, nnz = _random_csr(rng, n_rows, n_cols, lengths, np.int32)
    indices[::7] = n_cols - 1
    data = _values(rng, nnz, vtype)
    x_full = _values(rng, n_cols + 1, vtype)
    d, i, p = _upload(data, indices, indptr, vtype)
    plan = _capi.Plan(p, n_rows, nnz)
    lengths = np.diff(indptr.astype(np.int64))
    xt_full = to_torch(x_full, vtype, DEV)
    for off in (0, 1):
        x = x_full[off:off + n_cols]
        xt = xt_full[off:off + n_cols]
        assert (xt.data_ptr() % 4 == 0) == (off == 0 or vtype == "float32")
        y = _capi.spmv(d, i, p, xt, n_rows, n_cols, plan=plan)
        torch.cuda.synchronize()
        want = orc.csr_matvec(data, indices, indptr, x, n_rows, vtype=vtype)
        assert_rows_close(to_numpy(y), want, orc.row_scale(data, indices, indptr, x, n_rows, vtype=vtype),
                          vtype, f"x offset {off}",
                          exact=orc.row_exact(data, indices, indptr, x, n_rows, vtype=vtype),
                          lengths=lengths)
    plan.close()


def test_repeat_calls_bitwise_identical():
    rng = np.random.default_rng(9)
    lengths = np.clip(rng.zipf(1.7, 20000), 1, 30000)
    indices, indptr, nnz = _random_csr(rng, 20000, 20000, lengths, np.int32)
    d, i, p = _upload(_values(rng, nnz, "float32"), indices, indptr, "float32")
    x = to_torch(_values(rng, 20000, "float32"), None, DEV)
    plan = _capi.Plan(p, 20000, nnz)
    ys = [_capi.spmv(d, i, p, x, 20000, 20000, plan=plan).clone() for _ in range(3)]
    torch.cuda.synchronize()
    for y in ys[1:]:
        assert torch.equal(y, ys[0])


def test_plan_for_other_matrix_is_rejected():
    p1 = torch.tensor([0, 1, 2], dtype=torch.int32, device=DEV)
    plan = _capi.Plan(p1, 2, 2)
    d = torch.ones(3, device=DEV)
    i = torch.zeros(3, dtype=torch.int32, device=DEV)
    p2 = torch.tensor([0, 1, 3], dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError, match="different matrix"):
        _capi.spmv(d, i, p2, torch.ones(1, device=DEV), 2, 1, plan=plan)


# -- benchmark configurations --------------------------------------------------------

def _config(name, small):
    from mlx_sparse import synthetic as s

    if name == "laplacian":
        return s.laplacian_2d(128 if small else 1024), s.uniform(128 * 128 if small else 1 << 20, -1, 1, 1)
    if name == "random16":
        n = 1 << 16 if small else 1 << 22
        return s.random_fixed_row(n, 16, seed=0), s.uniform(n, -1, 1, 1)
    if name == "powerlaw":
        n = 1 << 16 if small else 1 << 21
        return s.power_law(n, 2.0, 200_000, seed=0), s.uniform(n, 0, 1, 1)
    if name == "poisson":
        g = 32 if small else 128
        return s.poisson_3d(g), s.uniform(g ** 3, -1, 1, 1)
    n = 1 << 16 if small else 1 << 20
    return s.banded(n, 32, 0.65, 70.0, seed=0), s.uniform(n, -1, 1, 1)


@pytest.mark.parametrize("name", ["laplacian", "random16", "powerlaw", "poisson", "banded"])
def test_configs_small(name):
    m, x = _config(name, small=True)
    vtypes = ["float32"] if name != "banded" else ["bfloat16", "float16", "complex64"]
    for vtype in vtypes:
        if vtype == "complex64":
            from mlx_sparse import synthetic as s

            data = s.complex_values(m, 3)
            xv = storage(x + 1j * x[::-1], vtype)
        else:
            data, xv = storage(m.data, vtype), storage(x, vtype)
        out, want = _check_spmv(data, m.indices, m.indptr, xv, m.shape[0], m.shape[1], vtype,
                                what=f"{name}/{vtype}")


@pytest.mark.parametrize("name", ["random16", "powerlaw"])
def test_configs_full_size(name):
    """The north-star matrices at their benchmark size, against the oracle."""
    m, x = _config(name, small=False)
    out, want = _check_spmv(m.data, m.indices, m.indptr, x, m.shape[0], m.shape[1], "float32",
                            what=f"{name}/full")
    if name == "random16":
        np.testing.assert_array_equal(out["plan"], want)
        d, i, p = _upload(m.data, m.indices, m.indptr, "float32")
        xt = to_torch(x, None, DEV)
        # the benchmark path: bound plan, AUTO picks LDS column panels; every
        # row is summed in stored order, so the result equals the oracle
        plan = _capi.Plan(p, m.shape[0], m.nnz, data=d, indices=i, n_cols=m.shape[1])
        info = plan.info()
        assert info.n_panels == 128 and info.n_slices == 0
        # every (panel, tile) segment is padded to a multiple of 4 entries
        assert info.panel_values % 4 == 0
        assert m.nnz <= info.panel_values < m.nnz + 4 * info.n_panels * info.n_tiles
        for _ in range(2):
            y = _capi.spmv(d, i, p, xt, m.shape[0], m.shape[1], plan=plan)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(to_numpy(y), want)
        plan.close()
        # XCD column slices on request
        plan = _capi.Plan(p, m.shape[0], m.nnz, data=d, indices=i, n_cols=m.shape[1],
                          slice_mode=_capi.SLICE_ON)
        assert plan.info().n_slices == 8
        y = _capi.spmv(d, i, p, xt, m.shape[0], m.shape[1], plan=plan)
        torch.cuda.synchronize()
        assert_rows_close(to_numpy(y), want,
                          orc.row_scale(m.data, m.indices, m.indptr, x, m.shape[0]), "float32",
                          "random16 sliced")


# -- XCD column slicing (bound plans) ------------------------------------------------

@pytest.mark.parametrize("vtype", VTYPES)
@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_sliced_plan_parity(vtype, index_dtype):
    rng = np.random.default_rng(31)
    n_rows, n_cols = 6000, 50000
    lengths = rng.integers(0, 40, n_rows)
    lengths[rng.random(n_rows) < 0.1] = 0
    lengths[[17, 2000, 5999]] = [3000, 9000, 700]  # long rows keep the unsliced path
    indices, indptr, nnz = _random_csr(rng, n_rows, n_cols, lengths, index_dtype)
    data, x = _values(rng, nnz, vtype), _values(rng, n_cols, vtype)
    want = orc.csr_matvec(data, indices, indptr, x, n_rows, vtype=vtype, n_threads=8)
    scale = orc.row_scale(data, indices, indptr, x, n_rows, vtype=vtype)
    d, i, p = _upload(data, indices, indptr, vtype)
    for W in (64, 512):  # W also sets which rows are long (> W values)
        plan = _capi.Plan(p, n_rows, nnz, W, data=d, indices=i, n_cols=n_cols,
                          slice_mode=_capi.SLICE_ON)
        info = plan.info()
        assert info.n_slices == 8 and info.slice_width * 8 >= n_cols
        for _ in range(2):  # partial sums are rewritten each call
            y = _capi.spmv(d, i, p, to_torch(x, vtype, DEV), n_rows, n_cols, plan=plan)
            torch.cuda.synchronize()
            assert_rows_close(to_numpy(y), want, scale, vtype, f"sliced {vtype} W={W}")
        plan.close()


def test_auto_selection_and_binding():
    from mlx_sparse import synthetic as s

    m = s.random_fixed_row(1 << 21, 16, seed=4)  # x = 8.4 MB, columns scattered
    d, i, p = _upload(m.data, m.indices, m.indptr, "float32")
    plan = _capi.Plan(p, m.shape[0], m.nnz, data=d, indices=i, n_cols=m.shape[1])
    assert plan.info().n_panels == 64 and plan.info().n_slices == 0
    x = s.uniform(m.shape[1], -1, 1, 5)
    y = _capi.spmv(d, i, p, to_torch(x, None, DEV), m.shape[0], m.shape[1], plan=plan)
    torch.cuda.synchronize()
    want = orc.csr_matvec(m.data, m.indices, m.indptr, x, m.shape[0], n_threads=8)
    np.testing.assert_array_equal(to_numpy(y), want)
    # a bound plan refuses other buffers
    d2 = d.clone()
    with pytest.raises(RuntimeError, match="bound to other"):
        _capi.spmv(d2, i, p, to_torch(x, None, DEV), m.shape[0], m.shape[1], plan=plan)
    plan.close()
    # a stencil with the same x size keeps the row blocks (its gathers are local)
    g = s.laplacian_2d(1 << 11)
    d, i, p = _upload(g.data, g.indices, g.indptr, "float32")
    plan = _capi.Plan(p, g.shape[0], g.nnz, data=d, indices=i, n_cols=g.shape[1])
    assert plan.info().n_slices == 0 and plan.info().n_panels == 0
    plan.close()
    # scattered, but too few short-row values to give each of the 256 compute
    # units a 65536-value pass-1 chunk: row blocks at x = 8.4 MB, XCD slices
    # from x = 16 MB on
    for n, kind in ((1 << 21, "blocks"), (1 << 22, "slices")):
        f = s.random_fixed_row(n, 2, seed=8)
        d, i, p = _upload(f.data, f.indices, f.indptr, "float32")
        plan = _capi.Plan(p, f.shape[0], f.nnz, data=d, indices=i, n_cols=f.shape[1])
        info = plan.info()
        assert info.n_panels == 0 and info.n_slices == (8 if kind == "slices" else 0), kind
        xf = s.uniform(f.shape[1], -1, 1, 9)
        y = _capi.spmv(d, i, p, to_torch(xf, None, DEV), f.shape[0], f.shape[1], plan=plan)
        torch.cuda.synchronize()
        want = orc.csr_matvec(f.data, f.indices, f.indptr, xf, f.shape[0], n_threads=8)
        assert_rows_close(to_numpy(y), want,
                          orc.row_scale(f.data, f.indices, f.indptr, xf, f.shape[0]), "float32",
                          f"auto {kind}")
        plan.close()


def test_sliced_through_api(gpu):
    from mlx_sparse import synthetic as s

    ms = gpu
    m = s.random_fixed_row(1 << 21, 16, seed=6)
    A = ms.csr_array((m.data, m.indices, m.indptr), shape=m.shape)
    assert A.plan().info()["n_panels"] == 64
    x = s.uniform(m.shape[1], -1, 1, 7)
    y = (A @ torch.from_numpy(x).to(DEV)).cpu().numpy()
    want = orc.csr_matvec(m.data, m.indices, m.indptr, x, m.shape[0], n_threads=8)
    np.testing.assert_array_equal(y, want)
    with ms.runtime.context(gpu_slice="on"):
        C = ms.csr_array((m.data, m.indices, m.indptr), shape=m.shape)
        assert C.plan().info()["n_slices"] == 8 and C.plan().info()["n_panels"] == 0
        assert_rows_close((C @ torch.from_numpy(x).to(DEV)).cpu().numpy(), want,
                          orc.row_scale(m.data, m.indices, m.indptr, x, m.shape[0]), "float32",
                          "sliced api")
    with ms.runtime.context(gpu_slice="off"):
        B = ms.csr_array((m.data, m.indices, m.indptr), shape=m.shape)
        assert B.plan().info()["n_slices"] == 0 and B.plan().info()["n_panels"] == 0
        np.testing.assert_array_equal((B @ torch.from_numpy(x).to(DEV)).cpu().numpy(), want)


# -- LDS column panels (bound plans) -------------------------------------------------

ACC_BYTES = {"float32": 4, "float16": 4, "bfloat16": 4, "complex64": 8}


def _assert_short_rows_equal(got, want, lengths, W, vtype, what):
    """Rows of at most W values are summed in stored order by both sides:
    equal bit for bit, the sign of zero included."""
    short = lengths <= W
    g, w = got[short], want[short]
    if vtype == "complex64":
        g, w = g.view(np.float32), w.view(np.float32)
    np.testing.assert_array_equal(g, w, err_msg=what)
    if vtype in ("float32", "complex64"):
        np.testing.assert_array_equal(np.signbit(g), np.signbit(w), err_msg=f"{what} (signed zero)")


@pytest.mark.parametrize("vtype", VTYPES)
@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_panel_plan_parity(vtype, index_dtype):
    rng = np.random.default_rng(41)
    n_rows, n_cols = 9000, 200_000
    lengths = rng.integers(0, 40, n_rows)
    lengths[rng.random(n_rows) < 0.1] = 0
    few = rng.random(n_rows) < 0.1
    lengths[few] = rng.integers(1, 5, int(few.sum()))  # the 1..4-value rule
    lengths[[17, 2000, 8999]] = [3000, 9000, 700]  # long rows: chunks of W values in the tiles
    indices, indptr, nnz = _random_csr(rng, n_rows, n_cols, lengths, index_dtype)
    data, x = _values(rng, nnz, vtype), _values(rng, n_cols, vtype)
    data[::53] = storage(np.array([-0.0]), vtype)[0] if vtype != "complex64" else data[::53]
    want = orc.csr_matvec(data, indices, indptr, x, n_rows, vtype=vtype, n_threads=8)
    scale = orc.row_scale(data, indices, indptr, x, n_rows, vtype=vtype)
    d, i, p = _upload(data, indices, indptr, vtype)
    xt = to_torch(x, vtype, DEV)
    for W in (64, 512):
        plan = _capi.Plan(p, n_rows, nnz, W, data=d, indices=i, n_cols=n_cols,
                          slice_mode=_capi.SLICE_PANELS)
        info = plan.info()
        PW = 131072 // ACC_BYTES[vtype]
        assert info.n_panels == -(-n_cols // PW) and info.panel_width == PW
        tb, te, seg = plan.export_panels()
        otb, ote, oseg = plan_oracle.panel_layout(indptr, indices, n_cols, ACC_BYTES[vtype], W)
        np.testing.assert_array_equal(tb, otb)
        np.testing.assert_array_equal(te, ote)
        np.testing.assert_array_equal(seg, oseg)
        assert info.panel_values == int(oseg[-1])
        for _ in range(2):  # products are rewritten each call
            y = _capi.spmv(d, i, p, xt, n_rows, n_cols, plan=plan)
            torch.cuda.synchronize()
            got = to_numpy(y)
            _assert_short_rows_equal(got, want, lengths, W, vtype, f"panels {vtype} W={W}")
            assert_rows_close(got, want, scale, vtype, f"panels {vtype} W={W}")
        # new values in the same buffer: the copy (long-row chunks included)
        # is regathered through the layout
        data2 = _values(rng, nnz, vtype)
        d.copy_(to_torch(data2, vtype, DEV))
        plan.refresh(d)
        want2 = orc.csr_matvec(data2, indices, indptr, x, n_rows, vtype=vtype, n_threads=8)
        scale2 = orc.row_scale(data2, indices, indptr, x, n_rows, vtype=vtype)
        got = to_numpy(_capi.spmv(d, i, p, xt, n_rows, n_cols, plan=plan))
        _assert_short_rows_equal(got, want2, lengths, W, vtype, f"panels refreshed {vtype} W={W}")
        assert_rows_close(got, want2, scale2, vtype, f"panels refreshed {vtype} W={W}")
        d.copy_(to_torch(data, vtype, DEV))
        plan.refresh(d)
        plan.close()


def test_panel_plan_small_and_degenerate():
    # a single panel, empty rows at both ends, one-value rows, n_cols not a
    # multiple of anything
    data = np.array([2.0, -1.0, 3.0, -0.0, 5.0], np.float32)
    indices = np.array([4, 0, 2, 1, 3], np.int32)
    indptr = np.array([0, 0, 1, 3, 4, 5, 5], np.int32)
    x = np.array([1.0, 7.0, -2.0, 0.5, 3.0], np.float32)
    d, i, p = _upload(data, indices, indptr, "float32")
    plan = _capi.Plan(p, 6, 5, data=d, indices=i, n_cols=5, slice_mode=_capi.SLICE_PANELS)
    assert plan.info().n_panels == 1 and plan.info().n_tiles == 1
    y = to_numpy(_capi.spmv(d, i, p, to_torch(x, None, DEV), 6, 5, plan=plan))
    want = orc.csr_matvec(data, indices, indptr, x, 6)
    np.testing.assert_array_equal(y, want)
    np.testing.assert_array_equal(np.signbit(y), np.signbit(want))  # -0.0 * 7 keeps its sign


def test_panel_plan_rejects_oversized_x():
    d = torch.ones(2, device=DEV)
    i = torch.zeros(2, dtype=torch.int32, device=DEV)
    p = torch.tensor([0, 1, 2], dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError, match="2048 panels"):
        _capi.Plan(p, 2, 2, data=d, indices=i, n_cols=2048 * 32768 + 1,
                   slice_mode=_capi.SLICE_PANELS)


@pytest.mark.parametrize("name", ["laplacian", "powerlaw", "banded"])
def test_panel_plan_on_configs(name):
    """Panels on request for the other benchmark matrices (AUTO keeps row
    blocks for them): short rows equal the oracle bit for bit."""
    m, x = _config(name, small=True)
    vtype = "bfloat16" if name == "banded" else "float32"
    data, xv = storage(m.data, vtype), storage(x, vtype)
    want = orc.csr_matvec(data, m.indices, m.indptr, xv, m.shape[0], vtype=vtype, n_threads=8)
    d, i, p = _upload(data, m.indices, m.indptr, vtype)
    plan = _capi.Plan(p, m.shape[0], m.nnz, data=d, indices=i, n_cols=m.shape[1],
                      slice_mode=_capi.SLICE_PANELS)
    assert plan.info().n_panels >= 1
    y = to_numpy(_capi.spmv(d, i, p, to_torch(xv, vtype, DEV), m.shape[0], m.shape[1], plan=plan))
    lengths = np.diff(m.indptr.astype(np.int64))
    _assert_short_rows_equal(y, want, lengths, 256, vtype, f"{name} panels")
    assert_rows_close(y, want, orc.row_scale(data, m.indices, m.indptr, xv, m.shape[0], vtype=vtype),
                      vtype, f"{name} panels", lengths=lengths, min_len_exempt=LONG_ROW_EXEMPT,
                      exact=orc.row_exact(data, m.indices, m.indptr, xv, m.shape[0], vtype=vtype))
