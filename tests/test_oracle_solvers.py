"""Pins the solver side of the CPU oracle (oracle_csr_cg, oracle_csr_pcg_jacobi)
before it checks the native and HIP solvers.

Checks chosen so that a plausible slip (a wrong sign in an update, a swapped
alpha/beta, a stale residual, a wrong status code) fails one of them:

- a hand-computed one-step solve and a diagonal system whose CG iteration
  count equals its number of distinct eigenvalues (Krylov closed form);
- dense float64 solves of SPD systems (2D Laplacian, random diagonally
  dominant), within the stopping tolerance scaled by the condition;
- SciPy's ``cg`` (float64) on the same systems: iteration counts within one;
- the reported residual equals ||b - A x|| of the returned x (recomputed in
  float64) to float32 rounding;
- the status rules of the reference loops (cg.cpp:122-145, 158-246;
  pcg.cpp:137-232): zero right-hand side, exact x0, maxiter = 0 and a short
  budget, non-finite input, an indefinite matrix, a non-positive
  preconditioner.
"""

from __future__ import annotations

import numpy as np
import pytest
import scipy.sparse as sp
import scipy.sparse.linalg as spla


def laplacian_2d(g):
    one = sp.diags([-1, 2, -1], [-1, 0, 1], shape=(g, g))
    A = (sp.kron(sp.identity(g), one) + sp.kron(one, sp.identity(g))).tocsr()
    A.sort_indices()
    return A.astype(np.float32)


def random_spd(n, seed, per_row=6):
    rng = np.random.default_rng(seed)
    rows = np.repeat(np.arange(n), per_row)
    cols = rng.integers(0, n, n * per_row)
    vals = rng.uniform(-1, 1, n * per_row)
    M = sp.coo_matrix((vals, (rows, cols)), shape=(n, n)).tocsr()
    S = M + M.T
    d = np.asarray(abs(S).sum(axis=1)).ravel() + 1.0
    A = (S + sp.diags(d)).tocsr()
    A.sum_duplicates()
    A.sort_indices()
    return A.astype(np.float32)


def _args(A, index_dtype=np.int32):
    return A.data.astype(np.float32), A.indices.astype(index_dtype), A.indptr.astype(index_dtype)


def _scipy_iterations(A, b, rtol):
    count = [0]
    spla.cg(A.astype(np.float64), b.astype(np.float64), rtol=rtol, atol=0.0, maxiter=10 * b.size,
            callback=lambda xk: count.__setitem__(0, count[0] + 1))
    return count[0]


def test_one_step_hand_computed(oracle):
    # A = [2], b = [4]: r0 = 4, alpha = 16 / 32 = 0.5, x = 2, r = 0
    x, info, res, its = oracle.csr_cg(np.array([2.0], np.float32), np.array([0], np.int32),
                                      np.array([0, 1], np.int32), np.array([4.0], np.float32))
    assert (x.tolist(), info, res, its) == ([2.0], 0, 0.0, 1)


def test_distinct_eigenvalues_bound_iterations(oracle):
    # diagonal A with 3 distinct values: CG ends in 3 steps (exact in theory;
    # float32 leaves a residual far below the tolerance)
    d = np.array([1.0, 1.0, 4.0, 4.0, 9.0, 9.0, 9.0], np.float32)
    n = d.size
    b = np.arange(1, n + 1, dtype=np.float32)
    x, info, res, its = oracle.csr_cg(d, np.arange(n, dtype=np.int32),
                                      np.arange(n + 1, dtype=np.int32), b, rtol=1e-6)
    assert info == 0 and its == 3
    np.testing.assert_allclose(x, b / d, rtol=1e-6)
    # Jacobi with the exact inverse diagonal: one step
    x, info, res, its = oracle.csr_pcg_jacobi(d, np.arange(n, dtype=np.int32),
                                              np.arange(n + 1, dtype=np.int32), b, 1.0 / d,
                                              rtol=1e-6)
    assert info == 0 and its == 1
    np.testing.assert_allclose(x, b / d, rtol=1e-6)


@pytest.mark.parametrize("name", ["laplacian", "random"])
@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_cg_against_dense_solve_and_scipy(oracle, name, index_dtype):
    A = laplacian_2d(24) if name == "laplacian" else random_spd(600, 3)
    n = A.shape[0]
    rng = np.random.default_rng(1)
    b = rng.standard_normal(n).astype(np.float32)
    rtol = 1e-6
    x, info, res, its = oracle.csr_cg(*_args(A, index_dtype), b, rtol=rtol)
    assert info == 0
    A64 = A.astype(np.float64)
    exact = np.linalg.solve(A64.toarray(), b.astype(np.float64))
    cond = np.linalg.cond(A64.toarray())
    assert np.linalg.norm(x - exact) <= 4 * cond * rtol * np.linalg.norm(exact)
    true_res = np.linalg.norm(b.astype(np.float64) - A64 @ x.astype(np.float64))
    # the recursive residual tracks the true one to float32 rounding
    assert abs(true_res - res) <= 1e-5 * np.linalg.norm(b) + 1e-3 * res
    assert res <= rtol * np.linalg.norm(b) * (1 + 1e-6)
    assert abs(its - _scipy_iterations(A, b, rtol)) <= 1


def test_pcg_jacobi_against_dense_solve(oracle):
    A = random_spd(500, 7)
    n = A.shape[0]
    # b large enough that |p.Ap| stays above the reference's absolute eps
    # floor until convergence (see test_pcg_near_zero_denominator_rule)
    b = (1e3 * np.random.default_rng(2).standard_normal(n)).astype(np.float32)
    inv_d = (1.0 / A.diagonal()).astype(np.float32)
    x, info, res, its = oracle.csr_pcg_jacobi(*_args(A), b, inv_d, rtol=1e-5)
    assert info == 0
    exact = np.linalg.solve(A.toarray().astype(np.float64), b.astype(np.float64))
    np.testing.assert_allclose(x, exact, rtol=0, atol=1e-3 * np.abs(exact).max())
    # Jacobi cannot take more steps than plain CG on a diagonally dominant matrix
    _, info_cg, _, its_cg = oracle.csr_cg(*_args(A), b, rtol=1e-5)
    assert info_cg == 0 and its <= its_cg


def test_status_rules(oracle):
    A = laplacian_2d(8)
    args = _args(A)
    n = A.shape[0]
    b = np.ones(n, np.float32)
    # zero right-hand side: tol = 0 and ||r0|| = 0 -> converged before a step
    x, info, res, its = oracle.csr_cg(*args, np.zeros(n, np.float32))
    assert (info, res, its) == (0, 0.0, 0) and not x.any()
    # exact x0 (for a b made from it)
    x0 = np.arange(n, dtype=np.float32) % 3
    bb = (A @ x0).astype(np.float32)
    x, info, res, its = oracle.csr_cg(*args, bb, x0=x0)
    assert (info, its) == (0, 0) and np.array_equal(x, x0)
    # maxiter = 0: status 1, nothing done; a short budget: status = maxiter
    x, info, res, its = oracle.csr_cg(*args, b, maxiter=0)
    assert (info, its) == (1, 0) and not x.any()
    np.testing.assert_allclose(res, np.sqrt(n), rtol=1e-6)
    x, info, res, its = oracle.csr_cg(*args, b, maxiter=3, rtol=1e-8)
    assert (info, its) == (3, 3)
    # non-finite right-hand side
    bad = b.copy()
    bad[5] = np.nan
    assert oracle.csr_cg(*args, bad)[1] == -3
    assert oracle.csr_pcg_jacobi(*args, bad, np.full(n, 0.25, np.float32))[1] == -3
    # indefinite: p.Ap = 0 on the first step -> breakdown -1 after 0 steps
    d = np.array([1.0, -1.0], np.float32)
    x, info, res, its = oracle.csr_cg(d, np.array([0, 1], np.int32), np.array([0, 1, 2], np.int32),
                                      np.array([1.0, 1.0], np.float32))
    assert (info, its) == (-1, 0)
    # non-positive preconditioner: r.z <= 0 at the start -> -2
    x, info, res, its = oracle.csr_pcg_jacobi(*args, b, np.full(n, -0.25, np.float32))
    assert (info, its) == (-2, 0)


def test_pcg_near_zero_denominator_rule(oracle):
    # the reference's PCG stops with -1 once |p.Ap| <= eps * max(1, |p||Ap|)
    # (pcg.cpp:171-176): with a tiny right-hand side that holds at step one
    A = laplacian_2d(6)
    n = A.shape[0]
    b = np.full(n, 1e-5, np.float32)
    x, info, res, its = oracle.csr_pcg_jacobi(*_args(A), b, np.full(n, 0.25, np.float32),
                                              rtol=1e-6)
    assert (info, its) == (-1, 0)
    # plain CG takes the double-precision rule (cg.cpp:174-197) and converges
    assert oracle.csr_cg(*_args(A), b, rtol=1e-6)[1] == 0
