"""Pins the BiCGSTAB and MINRES restatements of the CPU oracle
(oracle_csr_bicgstab, oracle_csr_minres) before they check the native CPU
loops and the device loops.

Checks chosen so that a plausible slip (a swapped alpha/omega, a wrong sign
in a recurrence, a missing true-residual check, a stale Givens rotation, a
wrong status code) fails one of them:

- hand-computed runs: BiCGSTAB on diag(1, 2) with b = (1, 1) converges in
  its second iteration through the s-check, at x = (1, 1/2); both solvers
  on c * I end in one iteration at x = b / c;
- Krylov closed forms: MINRES on a symmetric matrix with k distinct
  eigenvalues ends in k iterations;
- the reference's own test systems (tests/test_linalg_bicgstab.py:66-93,
  tests/test_linalg_minres.py:57-175): a 4x4 nonsymmetric system, a 6x6
  convection-diffusion system, a symmetric indefinite 4x4, a shifted SPD
  3x3, singular compatible and incompatible systems, with their bounds;
- float64 dense solves and SciPy's bicgstab / minres on larger systems;
- the reported residual against ||b - (A - shift I) x|| of the returned x;
- the status rules of the reference loops: zero right-hand side, exact x0,
  maxiter = 0, non-finite input, breakdown.
"""

from __future__ import annotations

import numpy as np
import pytest
import scipy.sparse as sp
import scipy.sparse.linalg as spla

from oracle import oracle as orc


def _csr(dense, index_dtype=np.int32):
    A = sp.csr_matrix(np.asarray(dense, dtype=np.float32))
    A.sort_indices()
    return (A.data.astype(np.float32), A.indices.astype(index_dtype),
            A.indptr.astype(index_dtype))


def _rel_residual(dense, x, b, shift=0.0):
    M = np.asarray(dense, np.float64) - shift * np.eye(len(b))
    return np.linalg.norm(M @ np.asarray(x, np.float64) - b) / max(np.linalg.norm(b), 1.0)


NONSYM = np.array([[5.0, 0.3, 0.0, 0.0], [-0.8, 4.0, 0.2, 0.0], [0.0, -0.5, 4.5, 0.1],
                   [0.2, 0.0, -0.4, 3.5]], np.float32)


def convection_diffusion(n=6):
    A = np.zeros((n, n), np.float32)
    for i in range(n):
        A[i, i] = 3.0 + 0.1 * i
        if i > 0:
            A[i, i - 1] = -1.15
        if i + 1 < n:
            A[i, i + 1] = -0.35
        if i + 2 < n:
            A[i, i + 2] = 0.08
    return A


def convection_2d(g, wind=0.4):
    """Upwinded 2D convection-diffusion: nonsymmetric, diagonally dominant."""
    one = sp.diags([-1 - wind, 2, -1 + wind], [-1, 0, 1], shape=(g, g))
    A = (sp.kron(sp.identity(g), one) + sp.kron(one, sp.identity(g))).tocsr()
    A.sort_indices()
    return A.astype(np.float32)


def laplacian_2d(g):
    one = sp.diags([-1, 2, -1], [-1, 0, 1], shape=(g, g))
    A = (sp.kron(sp.identity(g), one) + sp.kron(one, sp.identity(g))).tocsr()
    A.sort_indices()
    return A.astype(np.float32)


# -- BiCGSTAB ----------------------------------------------------------------------------

def test_bicgstab_hand_computed_two_steps():
    d, i, p = _csr(np.diag([1.0, 2.0]))
    x, info, res, its = orc.csr_bicgstab(d, i, p, np.ones(2, np.float32), rtol=1e-5)
    assert (info, its) == (0, 2)
    np.testing.assert_allclose(x, [1.0, 0.5], rtol=1e-6, atol=1e-7)
    assert res <= 1e-5 * np.sqrt(2)


def test_bicgstab_scaled_identity_one_step():
    d, i, p = _csr(3.0 * np.eye(5))
    b = np.arange(1, 6, dtype=np.float32)
    x, info, res, its = orc.csr_bicgstab(d, i, p, b)
    assert (info, its) == (0, 1)
    np.testing.assert_allclose(x, b / 3.0, rtol=1e-6)


@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_bicgstab_reference_nonsymmetric_system(index_dtype):
    b = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    x, info, _, _ = orc.csr_bicgstab(*_csr(NONSYM, index_dtype), b, rtol=1e-6, atol=1e-7,
                                     maxiter=64)
    assert info == 0
    np.testing.assert_allclose(x, np.linalg.solve(NONSYM, b), rtol=3e-5, atol=3e-5)
    assert _rel_residual(NONSYM, x, b) < 2e-6
    sx, sinfo = spla.bicgstab(sp.csr_matrix(NONSYM.astype(np.float64)), b.astype(np.float64),
                              rtol=1e-6, atol=1e-7, maxiter=64)
    assert sinfo == 0
    np.testing.assert_allclose(x, sx, rtol=8e-5, atol=8e-5)


def test_bicgstab_reference_convection_diffusion():
    A = convection_diffusion()
    b = np.linspace(0.25, 1.5, 6, dtype=np.float32)
    x, info, res, its = orc.csr_bicgstab(*_csr(A), b, rtol=1e-5, atol=1e-7, maxiter=80)
    assert info == 0 and its > 0
    assert _rel_residual(A, x, b) < 2e-5


def test_bicgstab_larger_system_against_dense_and_scipy():
    A = convection_2d(24)
    n = A.shape[0]
    b = np.random.default_rng(4).uniform(-1, 1, n).astype(np.float32)
    # float32 BiCGSTAB: r drifts from r_hat's direction near 1e-5 relative
    # residual, where the reference's absolute breakdown test (rho below
    # FLT_EPSILON) stops it with -1; 1e-4 is reached
    x, info, res, its = orc.csr_bicgstab(A.data, A.indices, A.indptr, b, rtol=1e-4)
    assert info == 0
    dense = A.toarray().astype(np.float64)
    want = np.linalg.solve(dense, b.astype(np.float64))
    cond = np.linalg.cond(dense)
    assert np.linalg.norm(x - want) <= 1e-4 * cond * np.linalg.norm(want)
    # the reported residual is the true residual of the returned x
    true = np.linalg.norm(b - dense @ x)
    assert abs(res - true) <= 1e-4 * max(true, 1e-12) + 1e-6 * np.linalg.norm(b)
    count = [0]
    spla.bicgstab(A.astype(np.float64), b.astype(np.float64), rtol=1e-4,
                  callback=lambda _: count.__setitem__(0, count[0] + 1))
    assert abs(its - count[0]) <= 2, (its, count[0])


def test_bicgstab_status_rules():
    d, i, p = _csr(NONSYM)
    x, info, res, its = orc.csr_bicgstab(d, i, p, np.zeros(4, np.float32))
    assert (info, its) == (0, 0) and not x.any()
    exact = np.linalg.solve(NONSYM, np.arange(1, 5, dtype=np.float32)).astype(np.float32)
    b = (NONSYM.astype(np.float64) @ exact).astype(np.float32)
    x, info, res, its = orc.csr_bicgstab(d, i, p, b, exact, rtol=1e-7, atol=1e-7)
    assert (info, its) == (0, 0)
    np.testing.assert_array_equal(x, exact)
    A = convection_diffusion()
    x, info, res, its = orc.csr_bicgstab(*_csr(A), np.linspace(-1, 1, 6, dtype=np.float32),
                                         maxiter=0)
    assert info > 0 and its == 0
    x, info, res, its = orc.csr_bicgstab(*_csr(A), np.linspace(-1, 1, 6, dtype=np.float32),
                                         maxiter=1, rtol=1e-9)
    assert info == 1 and its == 1
    bad = np.ones(4, np.float32)
    bad[2] = np.nan
    assert orc.csr_bicgstab(d, i, p, bad)[1] == -3


def test_bicgstab_singular_systems():
    dense = np.diag([0.0, 2.0, 3.0, 4.0]).astype(np.float32)
    b = np.array([0.0, 4.0, -3.0, 8.0], np.float32)
    x, info, _, _ = orc.csr_bicgstab(*_csr(dense), b, rtol=1e-6, atol=1e-7, maxiter=16)
    assert info == 0 and _rel_residual(dense, x, b) < 1e-7
    zero = np.zeros((3, 3), np.float32)
    data = np.zeros(3, np.float32)
    _, info, _, _ = orc.csr_bicgstab(data, np.arange(3, dtype=np.int32),
                                     np.arange(4, dtype=np.int32),
                                     np.array([1.0, 0.0, 0.0], np.float32), maxiter=8)
    assert info < 0


# -- MINRES ---------------------------------------------------------------------------------

INDEF = np.array([[2.0, 3.0, 0.0, 0.0], [3.0, 2.0, 0.5, 0.0], [0.0, 0.5, -1.5, 1.0],
                  [0.0, 0.0, 1.0, 2.5]], np.float32)


def test_minres_scaled_identity_one_step():
    d, i, p = _csr(-2.0 * np.eye(6))
    b = np.linspace(1, 2, 6, dtype=np.float32)
    x, info, res, its = orc.csr_minres(d, i, p, b)
    assert (info, its) == (0, 1)
    np.testing.assert_allclose(x, b / -2.0, rtol=1e-6)


@pytest.mark.parametrize("eigs", [[1.0, -3.0], [2.0, 5.0, -1.0], [1.0, 2.0, 3.0, -4.0]])
def test_minres_distinct_eigenvalue_count(eigs):
    """A symmetric matrix with k distinct eigenvalues: k iterations."""
    rng = np.random.default_rng(len(eigs))
    n = 40
    diag = np.array([eigs[j % len(eigs)] for j in range(n)], np.float64)
    Q, _ = np.linalg.qr(rng.standard_normal((n, n)))
    dense = ((Q * diag) @ Q.T).astype(np.float32)
    dense = (dense + dense.T) / 2
    b = rng.uniform(-1, 1, n).astype(np.float32)
    x, info, res, its = orc.csr_minres(*_csr(dense), b, rtol=1e-4)
    assert info == 0 and its == len(eigs), (its, eigs)


def test_minres_reference_indefinite_system():
    b = np.array([1.0, -2.0, 0.5, 3.0], np.float32)
    x, info, _, _ = orc.csr_minres(*_csr(INDEF), b, rtol=1e-6, atol=1e-7, maxiter=64)
    assert info == 0
    np.testing.assert_allclose(x, np.linalg.solve(INDEF, b), rtol=5e-5, atol=5e-5)
    sx, sinfo = spla.minres(sp.csr_matrix(INDEF.astype(np.float64)), b.astype(np.float64),
                            rtol=1e-6, maxiter=64)
    assert sinfo == 0
    np.testing.assert_allclose(x, sx, rtol=5e-5, atol=5e-5)
    assert _rel_residual(INDEF, x, b) < 2e-6


def test_minres_reference_shift_convention():
    dense = np.array([[4.0, 1.0, 0.0], [1.0, 2.5, 0.5], [0.0, 0.5, 3.0]], np.float32)
    b = np.array([1.0, -2.0, 0.5], np.float32)
    x, info, res, its = orc.csr_minres(*_csr(dense), b, shift=0.75, rtol=1e-6, atol=1e-7,
                                       maxiter=64)
    assert info == 0
    want = np.linalg.solve(dense - 0.75 * np.eye(3), b)
    np.testing.assert_allclose(x, want, rtol=2e-5, atol=2e-5)
    sx, _ = spla.minres(sp.csr_matrix(dense.astype(np.float64)), b.astype(np.float64),
                        shift=0.75, rtol=1e-6, maxiter=64)
    np.testing.assert_allclose(x, sx, rtol=2e-5, atol=2e-5)
    assert _rel_residual(dense, x, b, shift=0.75) < 2e-6


def test_minres_singular_compatible():
    dense = np.diag([0.0, 2.0, 3.0, -4.0]).astype(np.float32)
    b = np.array([0.0, 4.0, -3.0, 8.0], np.float32)
    x, info, _, _ = orc.csr_minres(*_csr(dense), b, rtol=1e-7, atol=1e-7, maxiter=32)
    assert info == 0 and np.all(np.isfinite(x))
    assert _rel_residual(dense, x, b) < 1e-7


def test_minres_larger_indefinite_against_dense_and_scipy():
    """A shifted 2D Laplacian with the shift inside its spectrum."""
    A = laplacian_2d(20)
    n = A.shape[0]
    shift = 1.3
    b = np.random.default_rng(8).uniform(-1, 1, n).astype(np.float32)
    x, info, res, its = orc.csr_minres(A.data, A.indices, A.indptr, b, rtol=1e-4, shift=shift)
    assert info == 0
    dense = A.toarray().astype(np.float64) - shift * np.eye(n)
    want = np.linalg.solve(dense, b.astype(np.float64))
    cond = np.linalg.cond(dense)
    assert np.linalg.norm(x - want) <= 1e-4 * cond * np.linalg.norm(want)
    true = np.linalg.norm(b - dense @ x)
    assert res <= 1e-4 * np.linalg.norm(b) * 1.0001
    assert abs(res - true) <= 1e-3 * true + 1e-6 * np.linalg.norm(b)
    sx, sinfo = spla.minres(A.astype(np.float64), b.astype(np.float64), shift=shift, rtol=1e-7)
    np.testing.assert_allclose(x, sx, atol=1e-4 * cond * np.abs(want).max())


def test_minres_status_rules():
    d, i, p = _csr(INDEF)
    x, info, res, its = orc.csr_minres(d, i, p, np.zeros(4, np.float32))
    assert (info, its, res) == (0, 0, 0.0)
    x, info, res, its = orc.csr_minres(d, i, p, np.ones(4, np.float32), maxiter=0)
    assert (info, its) == (1, 0)
    x, info, res, its = orc.csr_minres(d, i, p, np.ones(4, np.float32), maxiter=2, rtol=1e-12)
    assert (info, its) == (2, 2)
    bad = np.ones(4, np.float32)
    bad[1] = np.inf
    assert orc.csr_minres(d, i, p, bad)[1] == -3
    assert orc.csr_minres(d, i, p, np.ones(4, np.float32), shift=float("nan"))[1] == -3


# -- BiCGSTAB with a Jacobi preconditioner ---------------------------------------------
#
# oracle_csr_bicgstab_jacobi (reference src/preconditioners/bicgstab/
# bicgstab.cpp:140-521) is pinned by: M = I reproducing the unpreconditioned
# loop bit for bit; the closed form of a diagonal system (M = A^-1: one
# iteration); the reference's own test system with its bounds
# (tests/test_linalg_bicgstab.py:175-201, 313-333); SciPy's bicgstab with the
# same M (the same right-preconditioned recurrences) on a badly row-scaled
# system, where the preconditioner decides convergence; and the status rules
# in which the reference's preconditioned loop differs from the plain one.

def _inv_diag(A):
    d = np.asarray(A.diagonal() if sp.issparse(A) else np.diag(A), np.float32)
    return (np.float32(1.0) / d).astype(np.float32)


@pytest.mark.parametrize("system", ["nonsym", "convection", "conv2d"])
def test_bicgstab_jacobi_identity_matches_plain(system):
    if system == "nonsym":
        A, b, kw = NONSYM, np.array([1.0, 2.0, 3.0, 4.0], np.float32), dict(rtol=1e-6, atol=1e-7)
        args = _csr(A)
    elif system == "convection":
        A, b, kw = convection_diffusion(), np.linspace(0.25, 1.5, 6, dtype=np.float32), {}
        args = _csr(A)
    else:
        A = convection_2d(16)
        b = np.random.default_rng(2).uniform(-1, 1, A.shape[0]).astype(np.float32)
        kw = dict(rtol=1e-4)
        args = (A.data, A.indices, A.indptr)
    ones = np.ones(len(b), np.float32)
    xj, ij, rj, kj = orc.csr_bicgstab_jacobi(*args, b, ones, **kw)
    xp, ip, rp, kp = orc.csr_bicgstab(*args, b, **kw)
    assert (ij, kj) == (ip, kp) and ij == 0
    np.testing.assert_array_equal(xj, xp)
    assert rj == rp


def test_bicgstab_jacobi_diagonal_system_one_step():
    d = np.array([2.0, 0.5, 4.0, 8.0, 1.25], np.float32)
    b = np.array([1.0, -2.0, 3.0, 0.5, 7.0], np.float32)
    A = np.diag(d)
    x, info, res, its = orc.csr_bicgstab_jacobi(*_csr(A), b, _inv_diag(A), rtol=1e-6)
    assert (info, its) == (0, 1)
    np.testing.assert_allclose(x, b / d, rtol=2e-7)
    assert res <= 1e-6 * np.linalg.norm(b)
    # the plain loop needs one step per distinct eigenvalue (up to 5)
    _, info_p, _, its_p = orc.csr_bicgstab(*_csr(A), b, rtol=1e-6)
    assert info_p == 0 and its_p > 1


def test_bicgstab_jacobi_reference_system():
    b = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    x, info, res, its = orc.csr_bicgstab_jacobi(*_csr(NONSYM), b, _inv_diag(NONSYM), rtol=1e-4,
                                                atol=1e-7, maxiter=80)
    assert info == 0 and its > 0
    assert _rel_residual(NONSYM, x, b) < 2e-5
    np.testing.assert_allclose(x, np.linalg.solve(NONSYM, b), rtol=8e-5, atol=8e-5)


def test_bicgstab_jacobi_row_scaled_against_scipy():
    A0 = convection_2d(20)
    n = A0.shape[0]
    rng = np.random.default_rng(9)
    scale = np.float32(10.0) ** rng.uniform(-2, 2, n).astype(np.float32)
    A = (sp.diags(scale) @ A0).tocsr().astype(np.float32)
    A.sort_indices()
    b = (scale * rng.uniform(-1, 1, n)).astype(np.float32)
    inv = _inv_diag(A)
    x, info, res, its = orc.csr_bicgstab_jacobi(A.data, A.indices, A.indptr, b, inv, rtol=1e-5,
                                                maxiter=400)
    assert info == 0
    dense = A.toarray().astype(np.float64)
    want = np.linalg.solve(dense, b.astype(np.float64))
    cond = np.linalg.cond(np.diag(inv.astype(np.float64)) @ dense)
    assert np.linalg.norm(x - want) <= 4e-5 * cond * np.linalg.norm(want)
    assert abs(res - np.linalg.norm(b - dense @ x)) <= 1e-4 * res + 1e-6 * np.linalg.norm(b)
    count = [0]
    M = spla.LinearOperator((n, n), matvec=lambda v: inv.astype(np.float64) * v)
    sx, sinfo = spla.bicgstab(A.astype(np.float64), b.astype(np.float64), rtol=1e-5, M=M,
                              maxiter=400, callback=lambda _: count.__setitem__(0, count[0] + 1))
    assert sinfo == 0
    assert abs(its - count[0]) <= max(2, count[0] // 10), (its, count[0])
    # without the preconditioner the same budget is far from enough
    _, info_p, _, its_p = orc.csr_bicgstab(A.data, A.indices, A.indptr, b, rtol=1e-5,
                                           maxiter=400)
    assert info_p != 0 or its_p > 2 * its


def test_bicgstab_jacobi_status_rules():
    b = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    args = _csr(NONSYM)
    inv = _inv_diag(NONSYM)
    # zero right-hand side and exact x0: status 0 before the first iteration
    x, info, res, its = orc.csr_bicgstab_jacobi(*args, np.zeros(4, np.float32), inv)
    assert (info, its, res) == (0, 0, 0.0) and not x.any()
    exact = np.linalg.solve(NONSYM.astype(np.float64), b).astype(np.float32)
    bb = (NONSYM.astype(np.float64) @ exact).astype(np.float32)
    _, info, _, its = orc.csr_bicgstab_jacobi(*args, bb, inv, x0=exact, rtol=1e-3)
    assert (info, its) == (0, 0)
    # maxiter 0: the budget status (1) and the true residual of x0
    _, info, res, its = orc.csr_bicgstab_jacobi(*args, b, inv, maxiter=0)
    assert (info, its) == (1, 0) and res == np.float32(np.linalg.norm(b))
    # non-finite right-hand side: -3 before any residual (reported +inf),
    # where the plain loop reports the residual it computed
    bad = b.copy()
    bad[2] = np.nan
    _, info, res, its = orc.csr_bicgstab_jacobi(*args, bad, inv)
    assert (info, its) == (-3, 0) and res == np.inf
    _, info_p, res_p, _ = orc.csr_bicgstab(*args, bad)
    assert info_p == -3 and not np.isinf(res_p)
    # a non-finite preconditioner entry: p_hat is non-finite in iteration 1
    inv_bad = inv.copy()
    inv_bad[1] = np.inf
    _, info, res, its = orc.csr_bicgstab_jacobi(*args, b, inv_bad)
    assert (info, its) == (-3, 0) and res == np.float32(np.linalg.norm(b))
    # a budget that ends before convergence: status = maxiter, true residual
    x, info, res, its = orc.csr_bicgstab_jacobi(*args, b, inv, rtol=1e-7, atol=0.0, maxiter=1)
    assert (info, its) == (1, 1)
    assert res == pytest.approx(np.linalg.norm(b - NONSYM.astype(np.float64) @ x), rel=1e-5)


# -- MINRES with a Jacobi preconditioner -----------------------------------------------
#
# oracle_csr_minres_jacobi (reference src/preconditioners/minres/minres.cpp:
# 93-330): M = I reproduces the plain loop bit for bit; the closed form of
# preconditioned MINRES (k distinct eigenvalues of M^1/2 (A - shift I) M^1/2:
# k iterations); a diagonal system with M = A^-1 (one iteration, the
# reference's near-singular diagonal test, test_linalg_minres.py:182-201);
# the reference's system against SciPy's minres with the same M
# (test_linalg_minres.py:141-179); and the Jacobi status rules (-2 for a
# non-positive preconditioner or preconditioned product).

@pytest.mark.parametrize("shift", [0.0, 0.7])
def test_minres_jacobi_identity_matches_plain(shift):
    for A in (sp.csr_matrix(INDEF), laplacian_2d(12)):
        n = A.shape[0]
        b = np.random.default_rng(n).uniform(-1, 1, n).astype(np.float32)
        ones = np.ones(n, np.float32)
        args = (A.data.astype(np.float32), A.indices.astype(np.int32), A.indptr.astype(np.int32))
        got = orc.csr_minres_jacobi(*args, b, ones, rtol=1e-5, shift=shift)
        want = orc.csr_minres(*args, b, rtol=1e-5, shift=shift)
        assert got[1:] == want[1:]
        np.testing.assert_array_equal(got[0], want[0])


@pytest.mark.parametrize("eigs", [[1.0, -3.0], [2.0, 5.0, -1.0], [1.0, 2.0, 3.0, -4.0]])
def test_minres_jacobi_distinct_eigenvalue_count(eigs):
    rng = np.random.default_rng(len(eigs))
    n = 24
    Q, _ = np.linalg.qr(rng.standard_normal((n, n)))
    lam = np.array([eigs[j % len(eigs)] for j in range(n)])
    s = 10.0 ** rng.uniform(-1, 1, n)
    # A = S Q diag(lam) Q^T S, M = S^-2: M^1/2 A M^1/2 = Q diag(lam) Q^T
    dense = (s[:, None] * ((Q * lam) @ Q.T) * s[None, :])
    dense = ((dense + dense.T) / 2).astype(np.float32)
    inv = (1.0 / s ** 2).astype(np.float32)
    b = rng.uniform(-1, 1, n).astype(np.float32)
    x, info, res, its = orc.csr_minres_jacobi(*_csr(dense), b, inv, rtol=1e-4)
    assert (info, its) == (0, len(eigs))
    _, info_p, _, its_p = orc.csr_minres(*_csr(dense), b, rtol=1e-4, maxiter=200)
    assert its_p > len(eigs)


def test_minres_jacobi_diagonal_systems_one_step():
    for d in ([1.0e-8, 1.0, 2.0, 3.0], [2.0, -0.5, 4.0, 8.0, -1.25]):
        d = np.array(d, np.float32)
        dense = np.diag(d)
        b = np.linspace(-1.0, 2.0, len(d)).astype(np.float32)
        inv = (1.0 / np.abs(d)).astype(np.float32)
        x, info, res, its = orc.csr_minres_jacobi(*_csr(dense), b, inv, rtol=1e-6, atol=1e-7,
                                                  maxiter=8)
        assert info == 0 and np.all(np.isfinite(x))
        assert _rel_residual(dense, x, b) <= 1e-6
        # all positive: M A = I, one iteration; mixed signs: eigenvalues +-1
        assert its == (1 if np.all(d > 0) else 2)


def test_minres_jacobi_reference_system_against_scipy():
    dense = np.array([[2.0, 3.0, 0.0], [3.0, 2.0, 0.5], [0.0, 0.5, 4.0]], np.float32)
    b = np.array([1.0, -2.0, 0.5], np.float32)
    inv = (1.0 / np.diag(dense)).astype(np.float32)
    x, info, res, its = orc.csr_minres_jacobi(*_csr(dense), b, inv, rtol=1e-6, atol=1e-7,
                                              maxiter=64)
    assert info == 0
    np.testing.assert_allclose(x, np.linalg.solve(dense, b), rtol=5e-5, atol=5e-5)
    assert _rel_residual(dense, x, b) < 2e-6
    M = spla.LinearOperator(dense.shape, matvec=lambda v: inv.astype(np.float64) * v)
    sx, sinfo = spla.minres(sp.csr_matrix(dense.astype(np.float64)), b.astype(np.float64), M=M,
                            rtol=1e-6, maxiter=64)
    assert sinfo == 0
    np.testing.assert_allclose(x, sx, rtol=8e-5, atol=8e-5)


def test_minres_jacobi_larger_against_scipy():
    A = laplacian_2d(24)
    n = A.shape[0]
    rng = np.random.default_rng(6)
    s = (10.0 ** rng.uniform(-1, 1, n)).astype(np.float32)
    As = (sp.diags(s) @ A @ sp.diags(s)).tocsr().astype(np.float32)
    As.sort_indices()
    b = rng.uniform(-1, 1, n).astype(np.float32)
    inv = (1.0 / As.diagonal()).astype(np.float32)
    x, info, res, its = orc.csr_minres_jacobi(As.data, As.indices, As.indptr, b, inv, rtol=1e-5,
                                              shift=-0.3, maxiter=2000)
    assert info == 0
    dense = As.toarray().astype(np.float64) + 0.3 * np.eye(n)
    true = np.linalg.norm(b - dense @ x)
    # the reported residual is the float32 true residual of x
    assert abs(res - true) <= 1e-4 * true + 1e-6 * np.linalg.norm(b)
    # SciPy's iterates are the same preconditioned MINRES iterates (float64);
    # its own stopping test differs, so take the first iterate whose true
    # residual meets this loop's test
    iterates = []
    M = spla.LinearOperator((n, n), matvec=lambda v: inv.astype(np.float64) * v)
    spla.minres(As.astype(np.float64), b.astype(np.float64), shift=-0.3, M=M, rtol=1e-9,
                maxiter=2000, callback=lambda xk: iterates.append(xk.copy()))
    tol = 1e-5 * np.linalg.norm(b.astype(np.float64))
    first = next(k + 1 for k, xk in enumerate(iterates)
                 if np.linalg.norm(b - dense @ xk) <= tol)
    assert abs(its - first) <= 2, (its, first)
    _, _, _, its_p = orc.csr_minres(As.data, As.indices, As.indptr, b, rtol=1e-5, shift=-0.3,
                                    maxiter=2000)
    assert its_p > 2 * its


def test_minres_jacobi_status_rules():
    dense = np.diag(np.array([1.0, 2.0], np.float32))
    b = np.ones(2, np.float32)
    # a non-positive inverse diagonal entry: -2 before any iteration, also
    # when x0 already solves the system
    for inv in (np.array([1.0, -1.0], np.float32), np.array([1.0, 0.0], np.float32),
                np.array([1.0, np.nan], np.float32)):
        x, info, res, its = orc.csr_minres_jacobi(*_csr(dense), b, inv, maxiter=8)
        assert (info, its) == (-2, 0) and res == np.float32(np.sqrt(2.0))
        _, info, _, _ = orc.csr_minres_jacobi(*_csr(dense), b, inv,
                                              x0=np.array([1.0, 0.5], np.float32))
        assert info == -2
    # an infinite entry: the preconditioned product r.M r is not finite
    _, info, res, its = orc.csr_minres_jacobi(*_csr(dense), b, np.array([1.0, np.inf], np.float32))
    assert (info, its) == (-2, 0)
    # zero right-hand side, maxiter 0, a non-finite b
    inv = np.array([1.0, 0.5], np.float32)
    x, info, res, its = orc.csr_minres_jacobi(*_csr(dense), np.zeros(2, np.float32), inv)
    assert (info, its, res) == (0, 0, 0.0)
    _, info, res, its = orc.csr_minres_jacobi(*_csr(INDEF), np.ones(4, np.float32),
                                              np.ones(4, np.float32), maxiter=0)
    assert (info, its) == (1, 0) and res == np.float32(2.0)
    bad = b.copy()
    bad[0] = np.inf
    _, info, _, its = orc.csr_minres_jacobi(*_csr(dense), bad, inv)
    assert (info, its) == (-3, 0)
