"""Native CPU BiCGSTAB and MINRES (msx_csr_bicgstab_cpu, msx_csr_minres_cpu)
against the oracle through the C ABI - the same sequential loops, so x,
info, residual and iteration count agree bit for bit - and the drop-in API
``linalg.bicgstab`` / ``linalg.minres`` on the CPU device, with the
reference's own test systems and argument rules
(tests/test_linalg_bicgstab.py, tests/test_linalg_minres.py)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import _capi
from test_oracle_krylov import (INDEF, NONSYM, _csr, convection_2d, convection_diffusion,
                                laplacian_2d)


def _run(kind, A, b, index_dtype=np.int32, x0=None, **kw):
    d, i, p = (torch.from_numpy(np.ascontiguousarray(a))
               for a in (A.data.astype(np.float32), A.indices.astype(index_dtype),
                         A.indptr.astype(index_dtype)))
    return _capi.krylov(kind, d, i, p, torch.from_numpy(b),
                        None if x0 is None else torch.from_numpy(x0), **kw)


def _oracle(oracle, kind, A, b, index_dtype=np.int32, **kw):
    args = (A.data.astype(np.float32), A.indices.astype(index_dtype),
            A.indptr.astype(index_dtype), b)
    return (oracle.csr_bicgstab if kind == "bicgstab" else oracle.csr_minres)(*args, **kw)


def _same(got, want):
    x, info, res, its = got
    wx, winfo, wres, wits = want
    assert (info, its) == (winfo, wits)
    assert np.float32(res).tobytes() == np.float32(wres).tobytes()
    assert x.numpy().tobytes() == wx.tobytes()


@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_bicgstab_cpu_equals_oracle(oracle, index_dtype):
    import scipy.sparse as sp

    A = convection_2d(24)
    b = np.random.default_rng(4).uniform(-1, 1, A.shape[0]).astype(np.float32)
    for kw in ({"rtol": 1e-4}, {"rtol": 1e-6}, {"rtol": 1e-3, "atol": 0.05},
               {"maxiter": 5, "rtol": 1e-9}, {"maxiter": 0}):
        _same(_run("bicgstab", A, b, index_dtype, **kw),
              _oracle(oracle, "bicgstab", A, b, index_dtype, **kw))
    x0 = np.full(A.shape[0], 0.25, np.float32)
    _same(_run("bicgstab", A, b, x0=x0, rtol=1e-4), oracle.csr_bicgstab(
        A.data, A.indices, A.indptr, b, x0, rtol=1e-4))
    B = sp.csr_matrix(np.diag([1.0, 2.0]).astype(np.float32))
    _same(_run("bicgstab", B, np.ones(2, np.float32)),
          _oracle(oracle, "bicgstab", B, np.ones(2, np.float32)))


@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_minres_cpu_equals_oracle(oracle, index_dtype):
    A = laplacian_2d(20)
    b = np.random.default_rng(8).uniform(-1, 1, A.shape[0]).astype(np.float32)
    for kw in ({"rtol": 1e-4, "shift": 1.3}, {"rtol": 1e-5}, {"rtol": 1e-9, "maxiter": 9},
               {"maxiter": 0}, {"rtol": 1e-3, "atol": 0.02, "shift": -0.5}):
        _same(_run("minres", A, b, index_dtype, **kw),
              _oracle(oracle, "minres", A, b, index_dtype, **kw))


def test_cpu_status_cases_equal_oracle(oracle):
    import scipy.sparse as sp

    A = sp.csr_matrix(NONSYM)
    S = sp.csr_matrix(INDEF)
    bad = np.ones(4, np.float32)
    bad[2] = np.nan
    for kind, M in (("bicgstab", A), ("minres", S)):
        for b, kw in ((np.zeros(4, np.float32), {}), (np.ones(4, np.float32), {"maxiter": 0}),
                      (bad, {})):
            _same(_run(kind, M, b, **kw), _oracle(oracle, kind, M, b, **kw))
    zero = sp.csr_matrix((np.zeros(3, np.float32), np.arange(3), np.arange(4)), shape=(3, 3))
    got = _run("bicgstab", zero, np.array([1.0, 0.0, 0.0], np.float32), maxiter=8)
    assert got[1] < 0
    _same(got, _oracle(oracle, "bicgstab", zero, np.array([1.0, 0.0, 0.0], np.float32),
                       maxiter=8))


def test_api_on_cpu_reference_systems(cpu):
    ms = cpu
    from mlx_sparse import linalg

    def csr(dense):
        d, i, p = _csr(dense)
        return ms.csr_array((d, i, p), shape=dense.shape, canonical=True)

    b = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    x, info = linalg.bicgstab(csr(NONSYM), b, rtol=1e-6, atol=1e-7, maxiter=64)
    assert info == 0
    np.testing.assert_allclose(x.numpy(), np.linalg.solve(NONSYM, b), rtol=3e-5, atol=3e-5)
    A = convection_diffusion()
    x, info = linalg.bicgstab(csr(A), np.linspace(0.25, 1.5, 6, dtype=np.float32), tol=1e-5,
                              atol=1e-7, maxiter=80, return_info=True)
    assert info.solver == "bicgstab" and info.status == 0
    assert info.convergence_reason == "converged" and info.breakdown_reason is None
    assert info.rtol == 1e-5 and info.atol == 1e-7 and info.maxiter == 80
    with pytest.raises(ValueError, match="tol is a compatibility alias"):
        linalg.bicgstab(csr(A), np.ones(6, np.float32), rtol=1e-5, tol=1e-6)
    _, info = linalg.bicgstab(csr(A), np.ones(6, np.float32), maxiter=0, return_info=True)
    assert info.status > 0 and info.convergence_reason == "iteration_limit"
    assert info.iterations == 0
    bi = np.array([1.0, -2.0, 0.5, 3.0], np.float32)
    x, info = linalg.minres(csr(INDEF), bi, rtol=1e-6, atol=1e-7, maxiter=64)
    assert info == 0
    np.testing.assert_allclose(x.numpy(), np.linalg.solve(INDEF, bi), rtol=5e-5, atol=5e-5)
    dense = np.array([[4.0, 1.0, 0.0], [1.0, 2.5, 0.5], [0.0, 0.5, 3.0]], np.float32)
    x, info = linalg.minres(csr(dense), np.array([1.0, -2.0, 0.5], np.float32), shift=0.75,
                            rtol=1e-6, atol=1e-7, maxiter=64)
    assert info == 0
    np.testing.assert_allclose(x.numpy(), np.linalg.solve(dense - 0.75 * np.eye(3),
                                                          [1.0, -2.0, 0.5]), rtol=2e-5, atol=2e-5)
    with pytest.raises(ValueError, match="shift must be finite"):
        linalg.minres(csr(dense), np.ones(3, np.float32), shift=float("inf"))
    from mlx_sparse.linalg import preconditioners

    x, info = linalg.minres(csr(dense), np.ones(3, np.float32),
                            M=preconditioners.jacobi(csr(dense)), rtol=1e-6)
    assert info == 0
    x, info = linalg.bicgstab(csr(NONSYM), b, M=preconditioners.identity((4, 4)), rtol=1e-6)
    assert info == 0


def test_cpu_krylov_errors():
    d = torch.ones(1)
    i = torch.zeros(1, dtype=torch.int32)
    p = torch.tensor([0, 1], dtype=torch.int32)
    for kind in ("bicgstab", "minres"):
        with pytest.raises(RuntimeError, match="maxiter must be non-negative"):
            _capi.krylov(kind, d, i, p, torch.ones(1), maxiter=-1)


# -- BiCGSTAB with a Jacobi preconditioner ---------------------------------------------

def _row_scaled(g=16, seed=9):
    import scipy.sparse as sp

    A0 = convection_2d(g)
    rng = np.random.default_rng(seed)
    scale = np.float32(10.0) ** rng.uniform(-2, 2, A0.shape[0]).astype(np.float32)
    A = (sp.diags(scale) @ A0).tocsr().astype(np.float32)
    A.sort_indices()
    b = (scale * rng.uniform(-1, 1, A.shape[0])).astype(np.float32)
    return A, b


@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_bicgstab_jacobi_cpu_equals_oracle(oracle, index_dtype):
    """msx_csr_bicgstab_jacobi_cpu runs the oracle's loop bit for bit: x,
    status, residual and iterations, on converging solves, short budgets,
    the row-scaled system the preconditioner rescues, and the status cases
    where the Jacobi loop differs from the plain one (non-finite b: residual
    +inf; a non-finite inverse diagonal entry)."""
    import scipy.sparse as sp

    cases = []
    A = convection_2d(20)
    b = np.random.default_rng(4).uniform(-1, 1, A.shape[0]).astype(np.float32)
    inv = (1.0 / A.diagonal()).astype(np.float32)
    for kw in ({"rtol": 1e-4}, {"rtol": 1e-6}, {"maxiter": 3, "rtol": 1e-9}, {"maxiter": 0}):
        cases.append((A, b, inv, None, kw))
    cases.append((A, b, inv, np.full(A.shape[0], 0.25, np.float32), {"rtol": 1e-4}))
    As, bs = _row_scaled()
    cases.append((As, bs, (1.0 / As.diagonal()).astype(np.float32), None, {"rtol": 1e-5}))
    N = sp.csr_matrix(NONSYM)
    invn = (1.0 / np.diag(NONSYM)).astype(np.float32)
    bn = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    cases.append((N, bn, invn, None, {"rtol": 1e-4, "atol": 1e-7, "maxiter": 80}))
    bad_b = bn.copy()
    bad_b[1] = np.nan
    cases.append((N, bad_b, invn, None, {}))
    bad_inv = invn.copy()
    bad_inv[2] = np.inf
    cases.append((N, bn, bad_inv, None, {}))
    cases.append((N, np.zeros(4, np.float32), invn, None, {}))
    for M, rhs, iv, x0, kw in cases:
        args = (M.data.astype(np.float32), M.indices.astype(index_dtype),
                M.indptr.astype(index_dtype))
        got = _capi.krylov("bicgstab", *(torch.from_numpy(np.ascontiguousarray(a)) for a in args),
                           torch.from_numpy(rhs), None if x0 is None else torch.from_numpy(x0),
                           inv_diag=torch.from_numpy(iv), **kw)
        want = oracle.csr_bicgstab_jacobi(*args, rhs, iv, x0, **kw)
        _same(got, want)


def test_bicgstab_jacobi_api_on_cpu(cpu, oracle):
    """linalg.bicgstab(A, b, M=jacobi(A)) on the CPU device runs the Jacobi
    loop (the reference's test system and bounds,
    tests/test_linalg_bicgstab.py:175-201), equal to the oracle bit for
    bit; diagonal(...) and a plain inverse-diagonal tensor are the same
    preconditioner."""
    ms = cpu
    from mlx_sparse import linalg
    from mlx_sparse.linalg import preconditioners

    d, i, p = _csr(NONSYM)
    A = ms.csr_array((d, i, p), shape=NONSYM.shape, canonical=True)
    b = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    want = oracle.csr_bicgstab_jacobi(d, i, p, b, (1.0 / np.diag(NONSYM)).astype(np.float32),
                                      rtol=1e-4, atol=1e-7, maxiter=80)
    for M in (preconditioners.jacobi(A), preconditioners.diagonal(np.diag(NONSYM))):
        x, info = linalg.bicgstab(A, b, M=M, rtol=1e-4, atol=1e-7, maxiter=80, return_info=True)
        assert info.status == 0 and info.preconditioner in {"jacobi", "diagonal"}
        assert info.iterations == want[3]
        assert x.numpy().tobytes() == want[0].tobytes()
        np.testing.assert_allclose(x.numpy(), np.linalg.solve(NONSYM, b), rtol=8e-5, atol=8e-5)
    with pytest.raises(TypeError, match="sparse matrices"):
        linalg.bicgstab(A, b, M=A)


# -- MINRES with a Jacobi preconditioner -----------------------------------------------

@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_minres_jacobi_cpu_equals_oracle(oracle, index_dtype):
    """msx_csr_minres_jacobi_cpu runs the oracle's loop bit for bit, on
    scaled symmetric systems with and without a shift, short budgets and the
    -2 cases (a non-positive or non-finite inverse diagonal entry)."""
    import scipy.sparse as sp

    A = laplacian_2d(16)
    n = A.shape[0]
    rng = np.random.default_rng(6)
    s = (10.0 ** rng.uniform(-1, 1, n)).astype(np.float32)
    As = (sp.diags(s) @ A @ sp.diags(s)).tocsr().astype(np.float32)
    As.sort_indices()
    b = rng.uniform(-1, 1, n).astype(np.float32)
    inv = (1.0 / As.diagonal()).astype(np.float32)
    cases = [(As, b, inv, {"rtol": 1e-5}), (As, b, inv, {"rtol": 1e-5, "shift": -0.3}),
             (As, b, inv, {"maxiter": 4, "rtol": 1e-9}), (As, b, inv, {"maxiter": 0})]
    S = sp.csr_matrix(INDEF)
    b4 = np.array([1.0, -2.0, 0.5, 3.0], np.float32)
    cases.append((S, b4, np.full(4, 0.5, np.float32), {"rtol": 1e-6, "atol": 1e-7}))
    for bad in (np.array([0.5, -1.0, 0.5, 0.5], np.float32),
                np.array([0.5, np.nan, 0.5, 0.5], np.float32),
                np.array([0.5, np.inf, 0.5, 0.5], np.float32)):
        cases.append((S, b4, bad, {}))
    for M, rhs, iv, kw in cases:
        args = (M.data.astype(np.float32), M.indices.astype(index_dtype),
                M.indptr.astype(index_dtype))
        got = _capi.krylov("minres", *(torch.from_numpy(np.ascontiguousarray(a)) for a in args),
                           torch.from_numpy(rhs), None, inv_diag=torch.from_numpy(iv), **kw)
        want = oracle.csr_minres_jacobi(*args, rhs, iv, **kw)
        _same(got, want)


def test_minres_jacobi_api_on_cpu(cpu, oracle):
    """The reference's Jacobi MINRES tests through linalg.minres on the CPU
    device (tests/test_linalg_minres.py:141-231): the diagonal
    preconditioner's solution and bounds, the near-singular diagonal fixed
    by Jacobi, a non-SPD diagonal rejected with the reference's ValueError
    (and ending with -2 when the check is off), and the reference's
    TypeError for other preconditioners."""
    ms = cpu
    from mlx_sparse import linalg
    from mlx_sparse.linalg import preconditioners

    def csr(dense):
        d, i, p = _csr(dense)
        return ms.csr_array((d, i, p), shape=dense.shape, canonical=True)

    dense = np.array([[2.0, 3.0, 0.0], [3.0, 2.0, 0.5], [0.0, 0.5, 4.0]], np.float32)
    A = csr(dense)
    b = np.array([1.0, -2.0, 0.5], np.float32)
    x, info = linalg.minres(A, b, M=preconditioners.jacobi(A, check=True), rtol=1e-6, atol=1e-7,
                            maxiter=64, return_info=True)
    want = oracle.csr_minres_jacobi(*_csr(dense), b, (1.0 / np.diag(dense)).astype(np.float32),
                                    rtol=1e-6, atol=1e-7, maxiter=64)
    assert info.status == 0 and info.iterations == want[3]
    assert x.numpy().tobytes() == want[0].tobytes()
    np.testing.assert_allclose(x.numpy(), np.linalg.solve(dense, b), rtol=5e-5, atol=5e-5)

    near = np.diag(np.array([1.0e-8, 1.0, 2.0, 3.0], np.float32))
    An = csr(near)
    bn = np.array([1.0, -1.0, 0.5, 2.0], np.float32)
    x, info = linalg.minres(An, bn, M=preconditioners.jacobi(An, check=True), rtol=1e-6,
                            atol=1e-7, maxiter=8)
    assert info == 0 and np.all(np.isfinite(x.numpy()))
    assert np.linalg.norm(near.astype(np.float64) @ x.numpy() - bn) / np.linalg.norm(bn) <= 1e-7

    A2 = csr(np.diag(np.array([1.0, 2.0], np.float32)))
    M = preconditioners.diagonal(np.array([1.0, -1.0], np.float32), inverse=True)
    with pytest.raises(ValueError, match="symmetric positive-definite"):
        linalg.minres(A2, np.ones(2, np.float32), M=M)
    _, info = linalg.minres(A2, np.ones(2, np.float32), M=M, check_preconditioner=False,
                            maxiter=8)
    assert info < 0
    with pytest.raises(TypeError, match="identity, diagonal, and Jacobi"):
        linalg.minres(A2, np.ones(2, np.float32), M=lambda v: v)
