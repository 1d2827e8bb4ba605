"""Native CPU GMRES (msx_csr_gmres_cpu, the `use_cpu()` path) against the
oracle through the C ABI: the same sequential loop, so x, info, residual and
iteration count agree bit for bit; and the drop-in ``linalg.gmres`` API on
the CPU (argument checks, callbacks, SolverInfo) as the reference's tests
use it (tests/test_linalg_errors.py:280-360, test_linalg_native.py:105-115).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import _capi
from test_oracle_gmres import _csr, _random_nonsym, _scaled_nonsym


def _native(A, b, index_dtype=np.int32, x0=None, **kw):
    d, i, p = (torch.from_numpy(np.ascontiguousarray(a)) for a in
               (A.data.astype(np.float32), A.indices.astype(index_dtype),
                A.indptr.astype(index_dtype)))
    return _capi.gmres(d, i, p, torch.from_numpy(b),
                       None if x0 is None else torch.from_numpy(x0), **kw)


def _same(native, want):
    x, info, res, its = native
    wx, winfo, wres, wits = want
    assert (info, its) == (winfo, wits)
    assert np.float32(res).tobytes() == np.float32(wres).tobytes()
    assert x.numpy().tobytes() == wx.tobytes()


@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
@pytest.mark.parametrize("restart", [1, 4, 20, 60])
def test_gmres_cpu_equals_oracle(oracle, index_dtype, restart):
    A = _random_nonsym(400, seed=restart, shift=0.2)
    rng = np.random.default_rng(restart)
    b = rng.standard_normal(400).astype(np.float32)
    x0 = (0.1 * rng.standard_normal(400)).astype(np.float32)
    for kw in ({"rtol": 1e-6, "maxiter": 4000}, {"rtol": 1e-3, "atol": 0.5},
               {"rtol": 1e-9, "maxiter": 13}, {"rtol": 0.0, "maxiter": 0}):
        got = _native(A, b, index_dtype, x0=x0, restart=restart, **kw)
        want = oracle.csr_gmres(A.data, A.indices.astype(index_dtype),
                                A.indptr.astype(index_dtype), b, x0, restart=restart, **kw)
        _same(got, want)


@pytest.mark.parametrize("case", ["zero_rhs", "exact", "nan_b", "inf_x0", "nan_value",
                                  "breakdown", "hilbert"])
def test_gmres_cpu_status_cases_equal_oracle(oracle, case):
    dense = np.diag([2.0, 3.0, 4.0, 5.0]).astype(np.float32)
    b = np.ones(4, np.float32)
    x0 = None
    kw = {}
    if case == "zero_rhs":
        b = np.zeros(4, np.float32)
    elif case == "exact":
        x0 = (1.0 / np.diag(dense)).astype(np.float32)
    elif case == "nan_b":
        b[2] = np.nan
    elif case == "inf_x0":
        x0 = np.zeros(4, np.float32)
        x0[1] = np.inf
    elif case == "breakdown":
        b = np.array([1.0, 0.0, 1.0, 0.0], np.float32)  # an invariant subspace of dimension 2
        kw = {"restart": 4, "rtol": 1e-7}
    elif case == "hilbert":
        i = np.arange(5, dtype=np.float32)
        dense = (1.0 / (i[:, None] + i[None, :] + 1.0)).astype(np.float32)
        b = np.linspace(0.25, 1.25, 5, dtype=np.float32)
        kw = {"rtol": 1e-6, "atol": 1e-7, "restart": 5, "maxiter": 64}
    d, ix, ip = _csr(dense)
    if case == "nan_value":
        d = d.copy()
        d[0] = np.nan
    import scipy.sparse as sp
    A = sp.csr_matrix((d, ix, ip), shape=dense.shape)
    got = _native(A, b, x0=x0, **kw)
    want = oracle.csr_gmres(d, ix, ip, b, x0, **kw)
    _same(got, want)


def test_gmres_cpu_rejects_bad_arguments():
    d = torch.tensor([1.0])
    i = torch.tensor([0], dtype=torch.int32)
    p = torch.tensor([0, 1], dtype=torch.int32)
    b = torch.ones(1)
    with pytest.raises(RuntimeError, match="restart > 0"):
        _capi.gmres(d, i, p, b, restart=0)
    with pytest.raises(RuntimeError, match="restart > 0"):
        _capi.gmres(d, i, p, b, maxiter=-1)


# -- the drop-in API on the CPU --------------------------------------------------------------

def _spd_2x2(ms):
    return ms.csr_array((torch.tensor([4.0, 1.0, 1.0, 3.0]), torch.tensor([0, 1, 0, 1]),
                         torch.tensor([0, 2, 4])), shape=(2, 2), validate="full")


def test_linalg_gmres_matches_numpy_and_oracle(cpu, oracle):
    ms = cpu
    A = _spd_2x2(ms)
    b = torch.tensor([1.0, 2.0])
    x, info = ms.linalg.gmres(A, b, rtol=1e-6, atol=1e-7, maxiter=20)
    assert info == 0
    np.testing.assert_allclose(x.numpy(), np.linalg.solve([[4.0, 1.0], [1.0, 3.0]], [1.0, 2.0]),
                               rtol=5e-4, atol=5e-4)
    R = _random_nonsym(300, seed=5)
    M = ms.csr_array((torch.from_numpy(R.data), torch.from_numpy(R.indices.astype(np.int64)),
                      torch.from_numpy(R.indptr.astype(np.int64))), shape=R.shape)
    bb = np.random.default_rng(5).standard_normal(300).astype(np.float32)
    x, info = ms.linalg.gmres(M, torch.from_numpy(bb), restart=10, rtol=1e-6)
    wx, winfo, _, _ = oracle.csr_gmres(R.data, R.indices.astype(np.int64),
                                       R.indptr.astype(np.int64), bb, restart=10, rtol=1e-6,
                                       maxiter=3000)
    assert info == winfo == 0
    assert x.numpy().tobytes() == wx.tobytes()


def test_linalg_gmres_callbacks_and_info(cpu):
    ms = cpu
    A = _spd_2x2(ms)
    b = torch.tensor([1.0, 2.0])
    seen = []
    x, info = ms.linalg.gmres(A, b, callback=seen.append, maxiter=8)
    assert info == 0 and len(seen) == 1 and seen[0].shape == x.shape
    for callback_type in ("pr_norm", "legacy"):
        seen = []
        x, info = ms.linalg.gmres(A, b, callback=seen.append, callback_type=callback_type,
                                  return_info=True, maxiter=8)
        assert info.status == 0 and info.solver == "gmres" and info.restart == 2
        assert len(seen) == 1 and seen[0] == pytest.approx(info.residual_norm)
    with pytest.raises(TypeError, match="callable"):
        ms.linalg.gmres(A, b, callback=3, maxiter=8)


def test_linalg_gmres_argument_errors(cpu):
    ms = cpu
    A = _spd_2x2(ms)
    b = torch.tensor([1.0, 2.0])
    with pytest.raises(ValueError, match="callback_type"):
        ms.linalg.gmres(A, b, callback_type="invalid")
    with pytest.raises(ValueError, match="restart"):
        ms.linalg.gmres(A, b, restart=0)
    with pytest.raises(TypeError, match="sparse matrices"):
        ms.linalg.gmres(A, b, M=A)
    with pytest.raises(ValueError, match="preconditioner size"):
        ms.linalg.gmres(A, b, M=ms.linalg.preconditioners.diagonal(np.ones(3, np.float32)))
    x, info = ms.linalg.gmres(A, b, M=ms.linalg.preconditioners.identity(A), maxiter=8)
    assert info == 0
    with pytest.raises(ValueError, match="length"):
        ms.linalg.gmres(A, torch.ones(3))


# -- GMRES with a Jacobi preconditioner -------------------------------------------------------

@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
@pytest.mark.parametrize("restart", [1, 5, 20])
def test_gmres_jacobi_cpu_equals_oracle(oracle, index_dtype, restart):
    """msx_csr_gmres_jacobi_cpu runs the oracle's loop bit for bit: x,
    status, residual and iterations, on row-scaled systems (converging, a
    short budget, maxiter 0, a starting guess) and the Jacobi status rules
    (a non-finite inverse diagonal entry: -3 with an infinite residual;
    ||M r|| <= FLT_EPSILON: -1; a zero right-hand side: 0)."""
    A, inv = _scaled_nonsym(300, seed=restart)
    rng = np.random.default_rng(restart)
    b = rng.uniform(-1, 1, 300).astype(np.float32)
    x0 = (0.1 * rng.standard_normal(300)).astype(np.float32)
    cases = [(A, b, inv, None, {"rtol": 1e-5, "maxiter": 3000}),
             (A, b, inv, x0, {"rtol": 1e-4, "maxiter": 3000}),
             (A, b, inv, None, {"rtol": 1e-9, "maxiter": 7}),
             (A, b, inv, None, {"maxiter": 0})]
    bad = inv.copy()
    bad[7] = np.inf
    cases.append((A, b, bad, None, {}))
    cases.append((A, b, np.zeros(300, np.float32), None, {}))
    cases.append((A, np.zeros(300, np.float32), inv, None, {}))
    nan_b = b.copy()
    nan_b[3] = np.nan
    cases.append((A, nan_b, inv, None, {}))
    for M, rhs, iv, guess, kw in cases:
        kw = {"restart": restart, **kw}
        args = (M.data.astype(np.float32), M.indices.astype(index_dtype),
                M.indptr.astype(index_dtype))
        got = _capi.gmres(*(torch.from_numpy(np.ascontiguousarray(a)) for a in args),
                          torch.from_numpy(rhs), None if guess is None else torch.from_numpy(guess),
                          inv_diag=torch.from_numpy(iv), **kw)
        want = oracle.csr_gmres_jacobi(*args, rhs, iv, guess, **kw)
        _same(got, want)


def test_gmres_jacobi_cpu_rejects_bad_arguments():
    d = torch.tensor([1.0])
    i = torch.tensor([0], dtype=torch.int32)
    p = torch.tensor([0, 1], dtype=torch.int32)
    b = torch.ones(1)
    with pytest.raises(RuntimeError, match="csr_gmres_jacobi requires restart > 0"):
        _capi.gmres(d, i, p, b, restart=0, inv_diag=torch.ones(1))
    L = _capi.lib()
    res = _capi.SolverResult()
    st = L.msx_csr_gmres_jacobi_cpu(_capi.IT[torch.int32], 1, 1, _capi._p(d), _capi._p(i),
                                    _capi._p(p), _capi._p(b), _capi._p(b), None, _capi._p(b),
                                    1e-5, 0.0, 1, 1, _capi.ctypes.byref(res))
    assert st != 0 and "non-NULL" in _capi.last_error()


def test_native_gmres_jacobi_reference_tests(cpu):
    """The reference's native Jacobi GMRES tests through _native on the CPU
    device (tests/test_linalg_preconditioners.py:1600-1667): the true
    residual and a bounded iteration count, and a non-finite inverse
    diagonal entry ending with -3, no iterations, an infinite residual and
    x = x0."""
    ms = cpu
    from mlx_sparse import _native
    from mlx_sparse.linalg import preconditioners

    dense = np.array([[5.0, -1.0, 0.25, 0.0], [1.25, 4.0, -0.5, 0.25], [0.0, 0.75, 3.5, -1.0],
                      [0.5, 0.0, 1.0, 4.5]], np.float32)
    d, i, p = (torch.from_numpy(a) for a in _csr(dense))
    A = ms.csr_array((d, i, p), shape=dense.shape, canonical=True)
    b = np.array([2.0, -1.0, 0.25, 3.0], np.float32)
    M = preconditioners.jacobi(A)
    x, info, residual, iterations = _native.csr_gmres_jacobi(
        d, i, p, torch.from_numpy(b), torch.zeros(4), M.inverse_diagonal, A.shape, rtol=1e-6,
        atol=1e-7, restart=4, maxiter=32)
    true = np.linalg.norm(dense @ x.numpy() - b)
    assert int(info) == 0 and int(iterations) <= 8
    assert float(residual) == pytest.approx(true, abs=1e-5)
    assert true <= 2e-6 * max(np.linalg.norm(b), 1.0)

    A2 = _spd_2x2(ms)
    d2, i2, p2 = A2.buffers(torch.device("cpu"))
    x, info, residual, iterations = _native.csr_gmres_jacobi(
        d2, i2, p2, torch.tensor([1.0, 2.0]), torch.zeros(2), torch.tensor([np.inf, 1.0]),
        (2, 2), rtol=1e-6, atol=1e-8, restart=2, maxiter=8)
    assert int(info) == -3 and int(iterations) == 0 and np.isinf(float(residual))
    assert not x.numpy().any()


def test_linalg_gmres_jacobi_on_cpu(cpu, oracle):
    """linalg.gmres(A, b, M=jacobi(A)) on the CPU device: the reference's
    left-preconditioned test against SciPy
    (tests/test_linalg_preconditioners.py:1547-1597), equal to the oracle's
    Jacobi loop bit for bit; diagonal(...) and an inverse-diagonal tensor
    are the same preconditioner, and the identity runs the plain loop."""
    import scipy.sparse as sp
    import scipy.sparse.linalg as spla

    ms = cpu
    from mlx_sparse import linalg
    from mlx_sparse.linalg import preconditioners

    dense = np.array([[7.0, -2.0, 0.5, 0.0], [1.0, 5.5, -1.0, 0.25], [0.0, -0.5, 4.5, 1.0],
                      [0.25, 0.0, -0.75, 3.75]], np.float32)
    d, i, p = _csr(dense)
    A = ms.csr_array((torch.from_numpy(d), torch.from_numpy(i), torch.from_numpy(p)),
                     shape=dense.shape, canonical=True)
    b = np.array([1.0, -2.0, 0.5, 3.0], np.float32)
    inv = (1.0 / np.diag(dense)).astype(np.float32)
    want = oracle.csr_gmres_jacobi(d, i, p, b, inv, rtol=1e-6, atol=1e-7, restart=4, maxiter=32)
    Ms = spla.LinearOperator(dense.shape, matvec=lambda v: (1.0 / np.diag(dense)) * v,
                             dtype=np.float32)
    x_scipy, info_scipy = spla.gmres(sp.csr_matrix(dense), b, M=Ms, rtol=1e-6, atol=1e-7,
                                     restart=4, maxiter=32)
    assert info_scipy == 0
    for M in (preconditioners.jacobi(A), preconditioners.diagonal(np.diag(dense)),
              torch.from_numpy(inv)):
        x, info = linalg.gmres(A, b, M=M, rtol=1e-6, atol=1e-7, restart=4, maxiter=32,
                               return_info=True)
        assert info.status == 0 and info.iterations == want[3]
        assert x.numpy().tobytes() == want[0].tobytes()
        np.testing.assert_allclose(x.numpy(), x_scipy, rtol=2e-4, atol=2e-4)
        rel = np.linalg.norm(dense.astype(np.float64) @ x.numpy() - b) / np.linalg.norm(b)
        assert rel <= 2e-6
    x_id, info_id = linalg.gmres(A, b, M=preconditioners.identity(A), rtol=1e-6, maxiter=32)
    x_base, info_base = linalg.gmres(A, b, rtol=1e-6, maxiter=32)
    assert info_id == info_base == 0
    assert x_id.numpy().tobytes() == x_base.numpy().tobytes()
