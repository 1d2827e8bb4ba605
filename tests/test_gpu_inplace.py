"""Cached matrix state follows in-place updates of the values.

torch tensors are mutable, unlike the reference's arrays
(reference: mlx_sparse/_csr.py:33): after ``A.data`` changes in place (an
optimizer step on the values), a product must use the new values, whatever
the array cached - a bound plan's reordered copy (XCD slices, LDS panels),
device copies, the transpose and the adjoint.  Every result below is
checked against the oracle on the new values: bit for bit where both sides
sum a row in stored order (panel plans, row blocks of short rows, the
transpose's SpMV), within tol * sum|a*x| elsewhere.

Also: a plan is bound to the indptr buffer it was built from (a same-nnz
matrix with other rows is rejected), and a bound plan given new values
without a refresh is rejected.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import _capi
from _util import TORCH, assert_rows_close, storage, to_numpy, to_torch
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

DEV = "cuda"
VTYPES = ["float32", "float16", "bfloat16", "complex64"]


def _values(rng, n, vtype):
    v = rng.standard_normal(n)
    if vtype == "complex64":
        v = v + 1j * rng.standard_normal(n)
    return storage(v, vtype)


def _random_csr(rng, n_rows, n_cols, max_len, index_dtype=np.int32):
    lengths = rng.integers(0, max_len, n_rows)
    indptr = np.zeros(n_rows + 1, np.int64)
    np.cumsum(lengths, out=indptr[1:])
    indices = rng.integers(0, n_cols, int(indptr[-1]))
    return indices.astype(index_dtype), indptr.astype(index_dtype), lengths


def _short_rows_equal(got, want, lengths, W, vtype, what):
    short = lengths <= W
    g, w = got[short], want[short]
    if vtype == "complex64":
        g, w = g.view(np.float32), w.view(np.float32)
    np.testing.assert_array_equal(g, w, err_msg=what)


# -- the C ABI: msx_csr_plan_refresh ---------------------------------------------------

@pytest.mark.parametrize("vtype", VTYPES)
@pytest.mark.parametrize("mode", [_capi.SLICE_PANELS, _capi.SLICE_ON])
def test_plan_refresh_rewrites_the_copy(vtype, mode):
    rng = np.random.default_rng(11)
    n_rows, n_cols = 20_000, 300_000
    indices, indptr, lengths = _random_csr(rng, n_rows, n_cols, 40)
    lengths[5] = 0
    nnz = int(indptr[-1])
    data0, data1 = _values(rng, nnz, vtype), _values(rng, nnz, vtype)
    x = _values(rng, n_cols, vtype)
    d = to_torch(data0, vtype, DEV)
    i, p = to_torch(indices, None, DEV), to_torch(indptr, None, DEV)
    xt = to_torch(x, vtype, DEV)
    plan = _capi.Plan(p, n_rows, nnz, data=d, indices=i, n_cols=n_cols, slice_mode=mode)
    info = plan.info()
    assert (info.n_panels > 0) if mode == _capi.SLICE_PANELS else (info.n_slices == 8)
    for step, new in enumerate((data1, data0, data1)):
        # in place, same buffer
        d.copy_(to_torch(new, vtype, DEV))
        plan.refresh(d)
        y = to_numpy(_capi.spmv(d, i, p, xt, n_rows, n_cols, plan=plan))
        want = orc.csr_matvec(new, indices, indptr, x, n_rows, vtype=vtype, n_threads=8)
        scale = orc.row_scale(new, indices, indptr, x, n_rows, vtype=vtype)
        assert_rows_close(y, want, scale, vtype, f"refresh {step} {vtype}")
        if mode == _capi.SLICE_PANELS:
            _short_rows_equal(y, want, lengths, info.block_nnz, vtype, f"panels {step}")
    # a new buffer: rejected until the plan is refreshed with it, then bound to it
    d2 = to_torch(data0, vtype, DEV)
    with pytest.raises(RuntimeError, match="bound to other"):
        _capi.spmv(d2, i, p, xt, n_rows, n_cols, plan=plan)
    plan.refresh(d2)
    y = to_numpy(_capi.spmv(d2, i, p, xt, n_rows, n_cols, plan=plan))
    want = orc.csr_matvec(data0, indices, indptr, x, n_rows, vtype=vtype, n_threads=8)
    assert_rows_close(y, want, orc.row_scale(data0, indices, indptr, x, n_rows, vtype=vtype),
                      vtype, "rebound")
    with pytest.raises(RuntimeError, match="bound to other"):
        _capi.spmv(d, i, p, xt, n_rows, n_cols, plan=plan)
    plan.close()


@pytest.mark.parametrize("vtype", VTYPES)
@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_plan_refresh_with_long_rows(vtype, index_dtype):
    """A panel plan with virtual rows (W = 64: long rows cut into chunks,
    rows of 0..200 values, a few of thousands) refreshed twice: short rows
    equal the oracle bit for bit, every row within the tolerance; values
    that changed place would move the sums far past it."""
    rng = np.random.default_rng(23)
    n_rows, n_cols = 12_000, 250_000
    lengths = rng.integers(0, 200, n_rows)
    lengths[rng.random(n_rows) < 0.1] = 0
    lengths[[3, 7000, n_rows - 1]] = [4000, 9000, 1500]
    indptr = np.zeros(n_rows + 1, np.int64)
    np.cumsum(lengths, out=indptr[1:])
    nnz = int(indptr[-1])
    indices = rng.integers(0, n_cols, nnz).astype(index_dtype)
    indptr = indptr.astype(index_dtype)
    data0, data1 = _values(rng, nnz, vtype), _values(rng, nnz, vtype)
    x = _values(rng, n_cols, vtype)
    d = to_torch(data0, vtype, DEV)
    i, p = to_torch(indices, None, DEV), to_torch(indptr, None, DEV)
    xt = to_torch(x, vtype, DEV)
    plan = _capi.Plan(p, n_rows, nnz, 64, data=d, indices=i, n_cols=n_cols,
                      slice_mode=_capi.SLICE_PANELS)
    info = plan.info()
    assert info.n_panels > 0 and info.n_long_rows > 0
    for step, new in enumerate((data1, data0)):
        d.copy_(to_torch(new, vtype, DEV))
        plan.refresh(d)
        print(f"refresh long rows {vtype} {np.dtype(index_dtype).name} step {step}", flush=True)
        y = to_numpy(_capi.spmv(d, i, p, xt, n_rows, n_cols, plan=plan))
        want = orc.csr_matvec(new, indices, indptr, x, n_rows, vtype=vtype, n_threads=8)
        scale = orc.row_scale(new, indices, indptr, x, n_rows, vtype=vtype)
        assert_rows_close(y, want, scale, vtype, f"refresh long rows {step} {vtype}")
        _short_rows_equal(y, want, lengths, info.block_nnz, vtype, f"long rows {step}")
    plan.close()


def test_plan_is_bound_to_its_indptr_buffer():
    """Same n_rows and nnz, other rows: both plan kinds reject the matrix."""
    rng = np.random.default_rng(3)
    n_rows, n_cols = 5000, 4000
    indices, indptr, _ = _random_csr(rng, n_rows, n_cols, 20)
    nnz = int(indptr[-1])
    other = indptr.copy()
    other[1:-1] = np.sort(rng.integers(0, nnz, n_rows - 1))  # same nnz, other rows
    d = torch.ones(nnz, device=DEV)
    i = to_torch(indices, None, DEV)
    p, p2 = to_torch(indptr, None, DEV), to_torch(other, None, DEV)
    x = torch.ones(n_cols, device=DEV)
    for plan in (_capi.Plan(p, n_rows, nnz), _capi.Plan(p, n_rows, nnz, data=d, indices=i,
                                                        n_cols=n_cols)):
        with pytest.raises(RuntimeError, match="another indptr"):
            _capi.spmv(d, i, p2, x, n_rows, n_cols, plan=plan)
        st = _capi.lib().msx_csr_spmv(0, 0, n_rows, n_cols, nnz, d.data_ptr(), i.data_ptr(),
                                      p2.data_ptr(), x.data_ptr(),
                                      torch.empty(n_rows, device=DEV).data_ptr(), plan.ptr,
                                      _capi._stream())
        assert st == _capi.EINVAL
        y = _capi.spmv(d, i, p, x, n_rows, n_cols, plan=plan)  # its own indptr still works
        np.testing.assert_array_equal(to_numpy(y), np.diff(indptr).astype(np.float32))
        plan.close()


@pytest.mark.parametrize("vtype", VTYPES)
def test_transpose_positions_and_values(vtype):
    """msx_csr_transpose_positions lists, per entry of A^T, the position of
    A it holds: gathering A's values through it equals msx_csr_transpose and
    the oracle's transpose bit for bit (conjugated for A^H)."""
    rng = np.random.default_rng(5)
    n_rows, n_cols = 3000, 2500
    indices, indptr, _ = _random_csr(rng, n_rows, n_cols, 30)
    indices[7] = n_cols + 3  # out of range: dropped from the transpose
    nnz = int(indptr[-1])
    data = _values(rng, nnz, vtype)
    d = to_torch(data, vtype, DEV)
    i, p = to_torch(indices, None, DEV), to_torch(indptr, None, DEV)
    pos, ti, tp = _capi.transpose_positions(i, p, n_rows, n_cols)
    td, ti2, tp2 = _capi.transpose(d, i, p, n_rows, n_cols)
    kept = int(tp[-1].item())
    assert kept == nnz - 1
    assert torch.equal(tp, tp2) and torch.equal(ti[:kept], ti2[:kept])
    assert torch.all(pos[kept:] == -1)
    # the dropped values' tail is defined (zero bits, row 0) on every route,
    # so a regathered transpose equals a fresh one element for element
    assert torch.all(ti2[kept:] == 0) and torch.all(ti[kept:] == 0)
    out = torch.full_like(d, 7.0)
    _capi.transpose_values(d, pos, out)
    np.testing.assert_array_equal(to_numpy(out), to_numpy(td))
    ot, oi, op = orc.csr_transpose(data, indices, indptr, n_rows, n_cols, vtype=vtype)
    np.testing.assert_array_equal(to_numpy(out[:kept]), ot)
    np.testing.assert_array_equal(to_numpy(ti2[:kept]), oi)
    assert not to_numpy(out)[kept:].any()
    if vtype == "complex64":
        _capi.transpose_values(d, pos, out, conjugate=True)
        np.testing.assert_array_equal(to_numpy(out[:kept]), np.conj(ot))
        assert not to_numpy(out)[kept:].any()


# tile and bucket sizes of the two-pass regather, by value width
LAYOUT_SIZES = {2: (32768, 32768), 4: (32768, 16384), 8: (16384, 8192)}


def _check_layout(layout, pos, width):
    """The layout composes to the permutation: S position s (bucket s // D2)
    reads the slot src1[s] of tile src1[s] // D1, which holds the source p
    with slot1[p] == src1[s] % D1, and lands at bucket offset slot2[s] -
    so the destination (s // D2) * D2 + slot2[s] must list p in pos.  Also:
    every bucket's slot2 is a permutation of its offsets, a tile's slots
    are 0..count-1, and dropped entries (pos -1) read nothing."""
    D1, D2 = LAYOUT_SIZES[width]
    slot1 = to_numpy(layout[0]).view(np.uint16).astype(np.int64)
    src1 = to_numpy(layout[1]).view(np.uint32).astype(np.int64)
    slot2 = to_numpy(layout[2]).view(np.uint16).astype(np.int64)
    p = to_numpy(pos).astype(np.int64)
    n = p.size
    for b0 in range(0, n, D2):
        seg = slot2[b0:b0 + D2]
        assert np.array_equal(np.sort(seg), np.arange(seg.size)), b0
    used = slot1 != 0xFFFF
    assert np.array_equal(np.sort(np.flatnonzero(used)), np.sort(p[p >= 0]))
    addr = (np.flatnonzero(used) // D1) * D1 + slot1[used]
    for t0 in range(0, n, D1):
        k = slot1[t0:t0 + D1][used[t0:t0 + D1]]
        assert np.array_equal(np.sort(k), np.arange(k.size)), t0
    source_at = np.full(n, -1, np.int64)
    source_at[addr] = np.flatnonzero(used)
    valid = src1 != 0xFFFFFFFF
    assert int((~valid).sum()) == int((p < 0).sum())
    s = np.flatnonzero(valid)
    dest = (s // D2) * D2 + slot2[s]
    np.testing.assert_array_equal(p[dest], source_at[src1[s]])
    assert np.all(p[(np.flatnonzero(~valid) // D2) * D2 + slot2[~valid]] < 0)


def _bits(t, vtype):
    a = to_numpy(t)
    return a.view(np.float32).view(np.uint32) if vtype == "complex64" else a.view(
        np.uint16 if a.dtype.itemsize == 2 else np.uint32)


@pytest.mark.parametrize("vtype", VTYPES)
@pytest.mark.parametrize("n_rows,n_cols,max_len",
                         [(300, 200, 9), (9000, 7000, 30), (40000, 31000, 12),
                          (200000, 150000, 21)])
def test_transpose_layout_regather(vtype, n_rows, n_cols, max_len):
    """msx_csr_transpose_values_layout (two streaming passes through the
    layout of msx_csr_transpose_layout) writes exactly what the one-pass
    gather msx_csr_transpose_values writes - the oracle's transpose for the
    kept entries, zero bits for the dropped ones, conjugated on request -
    below one tile and across many tiles and buckets with ragged ends, on
    calls in a row that share the scratch (new values each time); the third
    call's values and output are views one element off their allocation, so
    the element-wise passes run instead of the quad ones."""
    rng = np.random.default_rng(n_rows + max_len)
    indices, indptr, _ = _random_csr(rng, n_rows, n_cols, max_len)
    indices[3] = n_cols + 1  # dropped from the transpose
    indices[-1] = -4
    nnz = int(indptr[-1])
    i, p = to_torch(indices, None, DEV), to_torch(indptr, None, DEV)
    pos, ti, tp = _capi.transpose_positions(i, p, n_rows, n_cols)
    kept = int(tp[-1].item())
    assert kept == nnz - 2
    width = {"float32": 4, "float16": 2, "bfloat16": 2, "complex64": 8}[vtype]
    layout = _capi.transpose_layout(pos, TORCH[vtype])
    if nnz <= 300000:
        _check_layout(layout, pos, width)
    scratch = torch.empty(nnz, dtype=TORCH[vtype], device=DEV)
    for trial in range(3):
        data = _values(rng, nnz, vtype)
        d = to_torch(data, vtype, DEV)
        want = torch.full_like(d, 7.0)
        _capi.transpose_values(d, pos, want)
        got = torch.full_like(d, 3.0)
        if trial == 2:  # misaligned views
            d = torch.cat([d[:1], d])[1:]
            got = torch.full((nnz + 1,), 3.0, dtype=d.dtype, device=DEV)[1:]
            assert d.data_ptr() % 16 != 0 and got.data_ptr() % 16 != 0
        _capi.transpose_values_layout(d, layout, got, scratch=scratch)
        np.testing.assert_array_equal(_bits(got, vtype), _bits(want, vtype), err_msg=f"trial {trial}")
        ot, _, _ = orc.csr_transpose(data, indices, indptr, n_rows, n_cols, vtype=vtype)
        np.testing.assert_array_equal(to_numpy(got[:kept]), ot)
        assert not to_numpy(got)[kept:].any()
        if vtype == "complex64":
            _capi.transpose_values_layout(d, layout, got, conjugate=True, scratch=scratch)
            np.testing.assert_array_equal(to_numpy(got[:kept]), np.conj(ot))
            assert not to_numpy(got)[kept:].any()


def test_refreshed_transpose_equals_a_fresh_one(gpu):
    """A matrix with an out-of-range column: after an in-place update of
    A.data, the cached A.T (values regathered through stored positions)
    equals a freshly built transpose of the new values in every element,
    the dropped values' tail included."""
    ms = gpu
    rng = np.random.default_rng(17)
    n_rows, n_cols = 2000, 1500
    indices, indptr, _ = _random_csr(rng, n_rows, n_cols, 20)
    indices[11] = n_cols + 5
    indices[300] = n_cols
    nnz = int(indptr[-1])
    data = _values(rng, nnz, "float32")
    A = ms.csr_array((torch.from_numpy(data), torch.from_numpy(indices), torch.from_numpy(indptr)),
                     shape=(n_rows, n_cols), validate=False)
    T0 = A.T
    assert int(T0.indptr[-1]) == nnz - 2
    _sgd(A, 0.25)
    T1 = A.T
    assert T1 is not T0
    fresh = ms.csr_array((A.data.detach().clone(), A.indices, A.indptr), shape=(n_rows, n_cols),
                         validate=False).T
    assert torch.equal(T1.data, fresh.data) and torch.equal(T1.indices, fresh.indices)
    assert torch.equal(T1.indptr, fresh.indptr)
    ot, oi, op = orc.csr_transpose(A.data.detach().cpu().numpy(), indices, indptr, n_rows, n_cols)
    np.testing.assert_array_equal(T1.data[:nnz - 2].cpu().numpy(), ot)
    assert not T1.data[nnz - 2:].cpu().numpy().any()


# -- the drop-in API: in-place updates of A.data ------------------------------------------

def _sgd(A, step):
    with torch.no_grad():
        A.data.mul_(0.5).add_(step)


def _check_forward_and_adjoint(ms, A, m_indices, m_indptr, shape, x, g, what, exact):
    n_rows, n_cols = shape
    data = A.data.detach().cpu().numpy()
    xn, gn = x.cpu().numpy(), g.cpu().numpy()
    y = (A @ x).cpu().numpy()
    want = orc.csr_matvec(data, m_indices, m_indptr, xn, n_rows, n_threads=8)
    if exact:
        np.testing.assert_array_equal(y, want, err_msg=f"{what}: A @ x")
    assert_rows_close(y, want, orc.row_scale(data, m_indices, m_indptr, xn, n_rows), "float32",
                      f"{what}: A @ x")
    # x.grad = A^T g, checked against the oracle's transpose and its SpMV
    xr = x.clone().requires_grad_()
    (A @ xr).backward(g)
    td, ti, tp = orc.csr_transpose(data, m_indices, m_indptr, n_rows, n_cols)
    want_t = orc.csr_matvec(td, ti, tp, gn, n_cols, n_threads=8)
    assert_rows_close(xr.grad.cpu().numpy(), want_t, orc.row_scale(td, ti, tp, gn, n_cols),
                      "float32", f"{what}: x.grad")
    # A.T follows the new values too; on a panel plan its SpMV sums every
    # row in stored order
    yt = (A.T @ g).cpu().numpy()
    if exact:
        np.testing.assert_array_equal(yt, want_t, err_msg=f"{what}: A.T @ g")
    assert_rows_close(yt, want_t, orc.row_scale(td, ti, tp, gn, n_cols), "float32",
                      f"{what}: A.T @ g")


@pytest.mark.parametrize("slice_mode", ["auto", "on"])
def test_inplace_update_on_a_bound_plan(gpu, slice_mode):
    """The panel plan AUTO builds for a 2M-row random matrix (16 per row) and
    the XCD-sliced plan: A @ x, x.grad and A.T @ g after SGD-style updates."""
    from mlx_sparse import runtime, synthetic

    ms = gpu
    m = synthetic.random_fixed_row(1 << 21, 16, seed=9)
    x = torch.from_numpy(synthetic.uniform(m.shape[1], -1, 1, seed=2)).to(DEV)
    g = torch.from_numpy(synthetic.uniform(m.shape[0], -1, 1, seed=3)).to(DEV)
    with runtime.context(gpu_slice=slice_mode, gpu_adjoint="auto"):
        A = ms.csr_array((m.data, m.indices, m.indptr), shape=m.shape)
        info = A.plan().info()
        if slice_mode == "auto":
            assert info["n_panels"] > 0
        else:
            assert info["n_slices"] == 8
        exact = slice_mode == "auto"  # panels sum every short row in stored order
        _check_forward_and_adjoint(ms, A, m.indices, m.indptr, m.shape, x, g, "initial", exact)
        plan = A.plan()
        for k in range(2):
            _sgd(A, 0.25 * (k + 1))
            _check_forward_and_adjoint(ms, A, m.indices, m.indptr, m.shape, x, g,
                                       f"after update {k}", exact)
            assert A.plan() is plan  # refreshed, not rebuilt


def test_inplace_update_trained_values_small_matrix(gpu):
    """Row blocks, gradients of the values themselves: three SGD steps on a
    requires-grad A.data under gpu_adjoint="auto" (atomic first, then the
    cached transpose, then the refreshed transpose); every step's forward
    and x.grad are checked against the oracle on that step's values."""
    from mlx_sparse import runtime

    ms = gpu
    rng = np.random.default_rng(17)
    n_rows, n_cols = 3000, 2000
    indices, indptr, lengths = _random_csr(rng, n_rows, n_cols, 30)
    data = torch.from_numpy(rng.standard_normal(int(indptr[-1])).astype(np.float32)).to(DEV)
    data.requires_grad_()
    A = ms.csr_array((data, indices, indptr), shape=(n_rows, n_cols))
    x = torch.from_numpy(rng.uniform(-1, 1, n_cols).astype(np.float32)).to(DEV)
    g = torch.from_numpy(rng.uniform(-1, 1, n_rows).astype(np.float32)).to(DEV)
    with runtime.context(gpu_adjoint="auto"):
        for step in range(3):
            vals = A.data.detach().cpu().numpy()
            xr = x.clone().requires_grad_()
            y = A @ xr
            want = orc.csr_matvec(vals, indices, indptr, x.cpu().numpy(), n_rows)
            np.testing.assert_array_equal(y.detach().cpu().numpy(), want)
            y.backward(g)
            td, ti, tp = orc.csr_transpose(vals, indices, indptr, n_rows, n_cols)
            gn = g.cpu().numpy()
            want_t = orc.csr_matvec(td, ti, tp, gn, n_cols)
            assert_rows_close(xr.grad.cpu().numpy(), want_t, orc.row_scale(td, ti, tp, gn, n_cols),
                              "float32", f"step {step}: x.grad")
            want_d = orc.csr_data_vjp(indices, indptr, x.cpu().numpy(), gn, n_rows, n_cols,
                                      int(indptr[-1]))
            np.testing.assert_array_equal(A.data.grad.cpu().numpy(), want_d)
            with torch.no_grad():
                A.data.sub_(0.5 * A.data.grad)
            A.data.grad = None


def test_inplace_update_of_a_host_array_used_on_the_gpu(gpu):
    """Values held on the host: the device copy is made again after an
    in-place update, and a tracked product with those values runs plan-free
    instead of failing on the plan's binding."""
    ms = gpu
    rng = np.random.default_rng(23)
    n_rows, n_cols = 1000, 800
    indices, indptr, _ = _random_csr(rng, n_rows, n_cols, 12)
    data = torch.from_numpy(rng.standard_normal(int(indptr[-1])).astype(np.float32))
    A = ms.CSRArray(data=data, indices=torch.from_numpy(indices), indptr=torch.from_numpy(indptr),
                    shape=(n_rows, n_cols))
    assert A.data.device.type == "cpu"
    x = torch.from_numpy(rng.uniform(-1, 1, n_cols).astype(np.float32)).to(DEV)
    for step in range(2):
        vals = A.data.numpy().copy()
        want = orc.csr_matvec(vals, indices, indptr, x.cpu().numpy(), n_rows)
        scale = orc.row_scale(vals, indices, indptr, x.cpu().numpy(), n_rows)
        np.testing.assert_array_equal((A @ x).cpu().numpy(), want)
        xr = x.clone().requires_grad_()
        # tracked with values copied from the host: the plan-free kernel
        # (several lanes per row) runs instead of the plan
        assert_rows_close((A @ xr).detach().cpu().numpy(), want, scale, "float32",
                          f"tracked step {step}")
        A.data.mul_(-2.0)
    # non-contiguous values with requires_grad: plan-free, same result
    base = torch.from_numpy(np.repeat(rng.standard_normal(int(indptr[-1])).astype(np.float32), 2))
    strided = base.to(DEV)[::2].requires_grad_()
    B = ms.CSRArray(data=strided, indices=torch.from_numpy(indices).to(DEV),
                    indptr=torch.from_numpy(indptr).to(DEV), shape=(n_rows, n_cols))
    vals = strided.detach().cpu().numpy()
    want = orc.csr_matvec(vals, indices, indptr, x.cpu().numpy(), n_rows)
    assert_rows_close((B @ x).detach().cpu().numpy(), want,
                      orc.row_scale(vals, indices, indptr, x.cpu().numpy(), n_rows), "float32",
                      "non-contiguous tracked values")


def test_hermitian_transpose_is_cached_and_follows_updates(gpu):
    ms = gpu
    rng = np.random.default_rng(29)
    n_rows, n_cols = 1500, 1200
    indices, indptr, _ = _random_csr(rng, n_rows, n_cols, 20)
    nnz = int(indptr[-1])
    for dtype in (torch.float32, torch.complex64):
        v = rng.standard_normal(nnz) + (1j * rng.standard_normal(nnz) if dtype == torch.complex64 else 0)
        A = ms.csr_array((torch.as_tensor(v).to(dtype), indices, indptr), shape=(n_rows, n_cols))
        H1 = A.H
        assert A.H is H1  # cached
        if dtype == torch.float32:
            assert A.T is H1  # real values: A^H is A^T
        with torch.no_grad():
            A.data.mul_(3.0)
        H2 = A.H
        vals = A.data.cpu().numpy()
        ot, oi, op = orc.csr_transpose(vals, indices, indptr, n_rows, n_cols)
        np.testing.assert_array_equal(H2.data.cpu().numpy(), np.conj(ot))
        np.testing.assert_array_equal(H2.indptr.cpu().numpy(), op)
        g = torch.as_tensor(rng.standard_normal(n_rows)).to(DEV, dtype)
        y = (H2 @ g).cpu().numpy()
        want = orc.csr_matvec(np.conj(ot), oi, op, g.cpu().numpy(), n_cols)
        assert_rows_close(y, want, orc.row_scale(np.conj(ot), oi, op, g.cpu().numpy(), n_cols),
                          "complex64" if dtype == torch.complex64 else "float32", "A.H @ g")
