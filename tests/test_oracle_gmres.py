"""Pins the restarted-GMRES restatement of the CPU oracle (oracle_csr_gmres,
over oracle_csr_arnoldi and its Givens least-squares solve) before it
checks the native CPU loop and the device loop.

Checks chosen so that a plausible slip (a dropped Gram-Schmidt pass, a
wrong sign in the projection, a transposed Hessenberg index, a rotation
applied to the wrong rows, a missing restart, a wrong status code) fails one
of them:

- the Arnoldi relation A V_k = V_{k+1} H_k and V^T V = I in float64 on
  the oracle's own output, H upper Hessenberg with a non-negative
  subdiagonal, and each H entry equal to <v_i, A v_j> (the two passes of
  modified Gram-Schmidt add up to the projection);
- Krylov closed forms: a matrix with k distinct eigenvalues (symmetric and
  not) is solved by one cycle of k steps and not by one of k - 1 (the
  reference tests convergence between cycles only); the Arnoldi
  factorisation of a v0 inside an invariant subspace of dimension m stops
  after m steps;
- the reference's own test systems and bounds
  (tests/test_linalg_native.py:105-115, tests/test_linalg_pathological.py:
  499-659): the 2x2 SPD system, the 3x3 system that converges on its last
  restart, the 5x5 nonsymmetric and 16-point convection-diffusion systems
  against SciPy and numpy, the Hilbert-like 5x5 that stops at its budget
  with a bounded residual;
- float64 dense solves and SciPy's gmres on larger random systems;
- the reported residual against ||b - A x|| of the returned x;
- the status rules of the reference loop: zero right-hand side, exact x0,
  maxiter = 0, a budget shorter than the solve, non-finite input, restart
  larger than n.
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


def _rel_residual(dense, x, b):
    return np.linalg.norm(np.asarray(dense, np.float64) @ np.asarray(x, np.float64) - b) / \
        max(np.linalg.norm(b), 1.0)


def _random_nonsym(n, seed, density=0.05, shift=None):
    rng = np.random.default_rng(seed)
    A = sp.random(n, n, density=density, random_state=rng, format="csr", dtype=np.float64)
    A.data = rng.standard_normal(A.nnz)
    d = np.abs(A).sum(axis=1).A1 + (1.0 if shift is None else shift)
    A = (A + sp.diags(d)).tocsr().astype(np.float32)
    A.sort_indices()
    return A


# -- Arnoldi ---------------------------------------------------------------------------------

@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
@pytest.mark.parametrize("k", [1, 5, 12])
def test_arnoldi_relation_and_orthonormality(index_dtype, k):
    A = _random_nonsym(60, seed=k)
    rng = np.random.default_rng(100 + k)
    v0 = rng.standard_normal(60).astype(np.float32)
    h, V, used = orc.csr_arnoldi(A.data, A.indices.astype(index_dtype),
                                 A.indptr.astype(index_dtype), v0, k)
    assert used == k
    H, V = h.astype(np.float64), V.astype(np.float64)
    Ad = A.toarray().astype(np.float64)
    # A V_k = V_{k+1} H_k; V orthonormal; V[:, 0] = v0 / ||v0||
    np.testing.assert_allclose(Ad @ V[:, :k], V @ H, atol=2e-5 * np.abs(Ad).max())
    np.testing.assert_allclose(V.T @ V, np.eye(k + 1), atol=1e-5)
    np.testing.assert_allclose(V[:, 0], v0 / np.linalg.norm(v0.astype(np.float64)), atol=1e-6)
    # upper Hessenberg, with h[j+1, j] = ||w|| >= 0 and every other entry a projection
    assert not np.tril(H, -2).any()
    assert np.all(np.diag(H, -1) >= 0)
    proj = V[:, :k].T @ Ad @ V[:, :k]
    np.testing.assert_allclose(np.triu(H[:k]), np.triu(proj), atol=2e-5 * np.abs(Ad).max())


def test_arnoldi_symmetric_matrix_gives_tridiagonal_h():
    rng = np.random.default_rng(4)
    B = rng.standard_normal((40, 40))
    S = (B + B.T).astype(np.float32)
    d, ix, ip = _csr(S)
    h, V, used = orc.csr_arnoldi(d, ix, ip, rng.standard_normal(40).astype(np.float32), 8)
    assert used == 8
    H = h.astype(np.float64)
    assert np.abs(np.triu(H[:8], 2)).max() <= 1e-4 * np.abs(H).max()
    np.testing.assert_allclose(np.diag(H[:8], 1), np.diag(H, -1)[:7], rtol=1e-4)


def test_arnoldi_stops_in_an_invariant_subspace():
    # v0 inside the span of three eigenvectors of a diagonal matrix
    diag = np.array([1.0, 2.0, 3.0, 4.0, 5.0, 6.0], np.float32)
    d, ix, ip = _csr(np.diag(diag))
    v0 = np.array([1.0, 0.0, 1.0, 0.0, 1.0, 0.0], np.float32)
    h, V, used = orc.csr_arnoldi(d, ix, ip, v0, 6)
    assert used == 3
    assert h[3, 2] <= np.finfo(np.float32).eps
    assert not V[:, 3:].any()  # no vector past the breakdown
    assert not h[:, 3:].any()


def test_arnoldi_zero_start_uses_the_first_unit_vector():
    d, ix, ip = _csr(np.diag([2.0, 3.0, 5.0]))
    h, V, used = orc.csr_arnoldi(d, ix, ip, np.zeros(3, np.float32), 2)
    np.testing.assert_array_equal(V[:, 0], [1.0, 0.0, 0.0])
    assert used == 1 and h[0, 0] == 2.0 and h[1, 0] == 0.0


# -- GMRES: closed forms ---------------------------------------------------------------------

@pytest.mark.parametrize("k", [2, 3, 4, 6])
def test_k_distinct_eigenvalues_take_k_steps(k):
    rng = np.random.default_rng(k)
    n = 30
    eig = np.repeat(np.arange(1, k + 1, dtype=np.float64) * 1.5, -(-n // k))[:n]
    Q, _ = np.linalg.qr(rng.standard_normal((n, n)))
    S = (Q @ np.diag(eig) @ Q.T).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    # the reference tests convergence only between cycles: one cycle of k
    # steps reaches the solution, one of k - 1 steps cannot
    x, info, res, its = orc.csr_gmres(*_csr(S), b, rtol=1e-5, restart=k, maxiter=k)
    assert info == 0 and its == k, (info, its)
    assert res <= 1e-5 * np.linalg.norm(b)
    x, info, res, its = orc.csr_gmres(*_csr(S), b, rtol=1e-5, restart=k - 1, maxiter=k - 1)
    assert info == k - 1 and its == k - 1
    assert res > 1e-3 * np.linalg.norm(b)


def test_diagonalizable_nonsymmetric_k_distinct_eigenvalues():
    rng = np.random.default_rng(12)
    n, k = 24, 3
    eig = np.repeat([1.0, -2.0, 4.0], n // k)
    P = np.eye(n) + 0.3 * rng.standard_normal((n, n)) / np.sqrt(n)  # cond(P) ~ 2
    A = (P @ np.diag(eig) @ np.linalg.inv(P)).astype(np.float32)
    assert np.abs(A - A.T).max() > 0.5
    b = rng.standard_normal(n).astype(np.float32)
    x, info, res, its = orc.csr_gmres(*_csr(A), b, rtol=1e-4, restart=k, maxiter=k)
    assert info == 0 and its == k, (info, its)
    x, info, res, its = orc.csr_gmres(*_csr(A), b, rtol=1e-4, restart=k - 1, maxiter=k - 1)
    assert info == k - 1 and res > 1e-2 * np.linalg.norm(b)


def test_gmres_one_restart_is_minimal_residual_steepest_descent():
    # GMRES(1): x1 = x0 + a r0 with a = <A r0, r0> / <A r0, A r0>
    A = np.array([[3.0, 1.0], [0.5, 2.0]], np.float32)
    b = np.array([1.0, 1.0], np.float32)
    x, info, res, its = orc.csr_gmres(*_csr(A), b, rtol=0.0, atol=0.0, restart=1, maxiter=1)
    r0 = b.astype(np.float64)
    Ar = A.astype(np.float64) @ r0
    a = Ar @ r0 / (Ar @ Ar)
    np.testing.assert_allclose(x, a * r0, rtol=1e-6)
    assert its == 1 and info == 1


# -- GMRES: the reference's systems and bounds ------------------------------------------------

def test_reference_spd_2x2_matches_numpy():
    dense = np.array([[4.0, 1.0], [1.0, 3.0]], np.float32)
    b = np.array([1.0, 2.0], np.float32)
    x, info, res, its = orc.csr_gmres(*_csr(dense), b, rtol=1e-6, atol=1e-7, maxiter=20)
    assert info == 0
    np.testing.assert_allclose(x, np.linalg.solve(dense, b), rtol=5e-4, atol=5e-4)


def test_reference_final_restart_reaches_true_tolerance():
    dense = np.array([[4.0, -1.0, 0.25], [0.5, 3.5, -0.75], [0.0, 0.4, 2.75]], np.float32)
    b = np.array([1.0, -2.0, 0.5], np.float32)
    x, info, res, its = orc.csr_gmres(*_csr(dense), b, rtol=1e-6, atol=1e-7, restart=3, maxiter=3)
    assert info == 0 and its == 3
    expected = np.linalg.solve(dense.astype(np.float64), b.astype(np.float64))
    np.testing.assert_allclose(x, expected, rtol=5e-5, atol=5e-5)
    assert _rel_residual(dense, x, b) <= 2e-6


def test_reference_nonsymmetric_diagonal_dominant_matches_scipy_and_numpy():
    dense = np.array([[5.0, -1.0, 0.5, 0.0, 0.0], [0.2, 4.5, -0.7, 0.4, 0.0],
                      [0.0, -0.3, 5.2, 1.1, 0.2], [0.0, 0.6, -0.2, 4.8, -1.0],
                      [0.1, 0.0, 0.5, -0.4, 3.9]], np.float32)
    b = np.array([1.0, -2.0, 0.5, 3.0, -1.5], np.float32)
    x, info, res, its = orc.csr_gmres(*_csr(dense), b, rtol=1e-6, atol=1e-7, restart=4, maxiter=40)
    xs, info_s = spla.gmres(sp.csr_array(dense), b, rtol=1e-6, atol=1e-7, restart=4, maxiter=40)
    assert info == 0 and info_s == 0
    expected = np.linalg.solve(dense.astype(np.float64), b.astype(np.float64))
    np.testing.assert_allclose(x, expected, rtol=5e-5, atol=5e-5)
    np.testing.assert_allclose(x, xs, rtol=5e-5, atol=5e-5)
    assert _rel_residual(dense, x, b) <= 2e-6


def test_reference_convection_diffusion_matches_scipy():
    n = 16
    diffusion, convection = np.float32(0.35), np.float32(1.15)
    A = sp.diags([-(diffusion + convection) * np.ones(n - 1, np.float32),
                  (2.0 * diffusion + convection + 1.0) * np.ones(n, np.float32),
                  -diffusion * np.ones(n - 1, np.float32)], offsets=[-1, 0, 1], format="csr",
                 dtype=np.float32)
    x_true = np.sin(np.linspace(0.15, 1.35, n, dtype=np.float32)).astype(np.float32)
    b = (A @ x_true).astype(np.float32)
    x, info, res, its = orc.csr_gmres(A.data, A.indices, A.indptr, b, rtol=1e-6, atol=1e-7,
                                      restart=8, maxiter=80)
    xs, info_s = spla.gmres(A, b, rtol=1e-6, atol=1e-7, restart=8, maxiter=80)
    assert info == 0 and info_s == 0
    np.testing.assert_allclose(x, xs, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(x, x_true, rtol=1e-4, atol=1e-4)
    assert _rel_residual(A.toarray(), x, b) <= 3e-6


def test_reference_hilbert_like_stops_at_budget_with_bounded_residual():
    n = 5
    i = np.arange(n, dtype=np.float32)
    dense = (1.0 / (i[:, None] + i[None, :] + 1.0)).astype(np.float32)
    b = np.linspace(0.25, 1.25, n, dtype=np.float32)
    x, info, res, its = orc.csr_gmres(*_csr(dense), b, rtol=1e-6, atol=1e-7, restart=5, maxiter=64)
    assert info == 64 and its == 64  # the reference's xfail: no convergence in float32
    rel = _rel_residual(dense, x, b)
    assert np.isfinite(rel) and rel < 2e-4


# -- GMRES: larger systems ---------------------------------------------------------------------

@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
@pytest.mark.parametrize("restart", [5, 20, 50])
def test_random_systems_against_dense_and_scipy(index_dtype, restart):
    A = _random_nonsym(300, seed=restart, shift=0.5)
    rng = np.random.default_rng(restart)
    b = rng.standard_normal(300).astype(np.float32)
    x, info, res, its = orc.csr_gmres(A.data, A.indices.astype(index_dtype),
                                      A.indptr.astype(index_dtype), b, rtol=1e-5,
                                      restart=restart, maxiter=3000)
    assert info == 0
    Ad = A.toarray().astype(np.float64)
    want = np.linalg.solve(Ad, b.astype(np.float64))
    cond = np.linalg.cond(Ad)
    assert np.linalg.norm(x - want) <= 4 * cond * 1e-5 * np.linalg.norm(want)
    xs, info_s = spla.gmres(A, b, rtol=1e-5, restart=restart, maxiter=3000)
    assert info_s == 0
    assert np.linalg.norm(x - xs) <= 8 * cond * 1e-5 * np.linalg.norm(want)
    # the reported residual is the true residual of the returned x
    true = np.linalg.norm(b - A.astype(np.float64) @ x.astype(np.float64))
    assert abs(res - true) <= 1e-3 * true + 1e-6 * np.linalg.norm(b)
    assert res <= 1e-5 * np.linalg.norm(b)


def test_restart_cycles_count_every_arnoldi_step():
    # a budget ending inside a cycle: iterations == maxiter, the last
    # cycle shortened to what is left, status = maxiter
    A = _random_nonsym(200, seed=3, shift=0.05)
    b = np.random.default_rng(3).standard_normal(200).astype(np.float32)
    x, info, res, its = orc.csr_gmres(A.data, A.indices, A.indptr, b, rtol=1e-12, restart=7,
                                      maxiter=17)
    assert info == 17 and its == 17
    true = np.linalg.norm(b - A.astype(np.float64) @ x.astype(np.float64))
    assert abs(res - true) <= 1e-3 * true


# -- GMRES: status rules -----------------------------------------------------------------------

def test_status_zero_rhs_and_exact_start():
    d, ix, ip = _csr(np.diag([2.0, 3.0, 4.0]))
    x, info, res, its = orc.csr_gmres(d, ix, ip, np.zeros(3, np.float32))
    assert (info, its, res) == (0, 0, 0.0) and not x.any()
    b = np.array([2.0, 3.0, 4.0], np.float32)
    x, info, res, its = orc.csr_gmres(d, ix, ip, b, np.ones(3, np.float32))
    assert (info, its, res) == (0, 0, 0.0)


def test_status_maxiter_zero():
    d, ix, ip = _csr(np.diag([2.0, 3.0, 4.0]))
    b = np.array([1.0, 1.0, 1.0], np.float32)
    x, info, res, its = orc.csr_gmres(d, ix, ip, b, maxiter=0)
    assert (info, its) == (1, 0)
    np.testing.assert_allclose(res, np.sqrt(3.0), rtol=1e-6)
    x, info, res, its = orc.csr_gmres(d, ix, ip, np.array([2.0, 3.0, 4.0], np.float32),
                                      np.ones(3, np.float32), maxiter=0)
    assert (info, its) == (0, 0)


@pytest.mark.parametrize("where", ["b", "x0", "rtol"])
def test_status_nonfinite_inputs(where):
    d, ix, ip = _csr(np.diag([2.0, 3.0, 4.0]))
    b = np.ones(3, np.float32)
    x0 = np.zeros(3, np.float32)
    rtol = 1e-5
    if where == "b":
        b[1] = np.nan
    elif where == "x0":
        x0[2] = np.inf
    else:
        rtol = float("inf")
    x, info, res, its = orc.csr_gmres(d, ix, ip, b, x0, rtol=rtol)
    assert info == -3 and its == 0 and res == np.inf
    np.testing.assert_array_equal(x, x0)


def test_status_nonfinite_matrix_value():
    d, ix, ip = _csr(np.diag([2.0, 3.0, 4.0]))
    d = d.copy()
    d[1] = np.nan
    x, info, res, its = orc.csr_gmres(d, ix, ip, np.ones(3, np.float32))
    assert info == -3 and its == 0 and np.isnan(res)


def test_restart_larger_than_n_clamps_to_n():
    A = _random_nonsym(12, seed=8, density=0.4)
    b = np.random.default_rng(8).standard_normal(12).astype(np.float32)
    x, info, res, its = orc.csr_gmres(A.data, A.indices, A.indptr, b, rtol=1e-5, restart=100,
                                      maxiter=100)
    assert info == 0 and its <= 12 + 12  # one full cycle of n steps, then at most one more
    assert _rel_residual(A.toarray(), x, b) <= 1e-5 * 1.01


# -- GMRES with a Jacobi preconditioner ------------------------------------------------
#
# oracle_csr_arnoldi_jacobi / oracle_csr_gmres_jacobi (reference
# src/preconditioners/gmres/gmres.cpp:342-748) are pinned by: M = I
# reproducing the plain loops bit for bit; the Arnoldi relation of M A; the
# Krylov closed form for M A with k distinct eigenvalues; the reference's own
# tests (tests/test_linalg_preconditioners.py:1600-1667); the Jacobi status
# rules (||M r|| <= FLT_EPSILON: -1; a non-finite inverse diagonal: -3 with an
# infinite residual).

def _scaled_nonsym(n, seed, decades=1.0):
    """_random_nonsym with rows scaled by 10^U[-decades, decades]; over two
    decades the float32 true residual stagnates near 2e-5 relative."""
    A0 = _random_nonsym(n, seed)
    rng = np.random.default_rng(seed + 1)
    d = (10.0 ** rng.uniform(-decades, decades, n)).astype(np.float32)
    A = (sp.diags(d) @ A0).tocsr().astype(np.float32)
    A.sort_indices()
    return A, (1.0 / A.diagonal()).astype(np.float32)


@pytest.mark.parametrize("restart", [3, 10])
def test_gmres_jacobi_identity_matches_plain(restart):
    A = _random_nonsym(80, seed=restart)
    b = np.random.default_rng(restart).uniform(-1, 1, 80).astype(np.float32)
    ones = np.ones(80, np.float32)
    got = orc.csr_gmres_jacobi(A.data, A.indices, A.indptr, b, ones, rtol=1e-5, restart=restart)
    want = orc.csr_gmres(A.data, A.indices, A.indptr, b, rtol=1e-5, restart=restart)
    assert got[1:] == want[1:]
    np.testing.assert_array_equal(got[0], want[0])
    v0 = np.random.default_rng(1).standard_normal(80).astype(np.float32)
    hj, Vj, uj = orc.csr_arnoldi_jacobi(A.data, A.indices, A.indptr, ones, v0, 7)
    hp, Vp, up = orc.csr_arnoldi(A.data, A.indices, A.indptr, v0, 7)
    assert uj == up == 7
    np.testing.assert_array_equal(hj, hp)
    np.testing.assert_array_equal(Vj, Vp)


def test_arnoldi_jacobi_relation():
    A, inv = _scaled_nonsym(60, seed=3, decades=2.0)
    v0 = np.random.default_rng(2).standard_normal(60).astype(np.float32)
    k = 8
    h, V, used = orc.csr_arnoldi_jacobi(A.data, A.indices, A.indptr, inv, v0, k)
    assert used == k
    MA = np.diag(inv.astype(np.float64)) @ A.toarray().astype(np.float64)
    H, V = h.astype(np.float64), V.astype(np.float64)
    np.testing.assert_allclose(MA @ V[:, :k], V @ H, atol=3e-5 * np.abs(MA).max())
    np.testing.assert_allclose(V.T @ V, np.eye(k + 1), atol=1e-5)
    # the plain factorisation is of A, not M A
    hp, _, _ = orc.csr_arnoldi(A.data, A.indices, A.indptr, v0, k)
    assert np.abs(hp - h).max() > 1e-2


@pytest.mark.parametrize("k", [2, 3, 5])
def test_gmres_jacobi_k_distinct_eigenvalues(k):
    rng = np.random.default_rng(k)
    n = 30
    Q, _ = np.linalg.qr(rng.standard_normal((n, n)))
    lam = np.array([[1.0, 3.0, -2.0, 5.0, 0.5][j % k] for j in range(n)])
    B = (Q * lam) @ Q.T
    d = 10.0 ** rng.uniform(-1, 1, n)
    dense = (B / d[:, None]).astype(np.float32)  # M A = B for M = diag(d)
    inv = d.astype(np.float32)
    b = rng.uniform(-1, 1, n).astype(np.float32)
    x, info, res, its = orc.csr_gmres_jacobi(*_csr(dense), b, inv, rtol=1e-4, restart=k,
                                             maxiter=k)
    assert (info, its) == (0, k)
    _, info1, _, _ = orc.csr_gmres_jacobi(*_csr(dense), b, inv, rtol=1e-4, restart=k - 1,
                                          maxiter=k - 1)
    assert info1 == k - 1


def test_gmres_jacobi_reference_tests():
    A = np.array([[5.0, -1.0, 0.25, 0.0], [1.25, 4.0, -0.5, 0.25], [0.0, 0.75, 3.5, -1.0],
                  [0.5, 0.0, 1.0, 4.5]], np.float32)
    b = np.array([2.0, -1.0, 0.25, 3.0], np.float32)
    inv = (1.0 / np.diag(A)).astype(np.float32)
    x, info, res, its = orc.csr_gmres_jacobi(*_csr(A), b, inv, rtol=1e-6, atol=1e-7, restart=4,
                                             maxiter=32)
    true = np.linalg.norm(A.astype(np.float64) @ x - b)
    assert info == 0 and its <= 8
    assert res == pytest.approx(true, abs=1e-5)
    assert true <= 2e-6 * max(np.linalg.norm(b), 1.0)
    spd = np.array([[4.0, 1.0], [1.0, 3.0]], np.float32)
    x, info, res, its = orc.csr_gmres_jacobi(*_csr(spd), np.array([1.0, 2.0], np.float32),
                                             np.array([np.inf, 1.0], np.float32), rtol=1e-6,
                                             atol=1e-8, restart=2, maxiter=8)
    assert (info, its) == (-3, 0) and np.isinf(res) and not x.any()


def test_gmres_jacobi_row_scaled_against_dense():
    A, inv = _scaled_nonsym(200, seed=11)
    b = np.random.default_rng(5).uniform(-1, 1, 200).astype(np.float32)
    x, info, res, its = orc.csr_gmres_jacobi(A.data, A.indices, A.indptr, b, inv, rtol=1e-5,
                                             restart=20, maxiter=400)
    assert info == 0
    dense = A.toarray().astype(np.float64)
    want = np.linalg.solve(dense, b.astype(np.float64))
    cond = np.linalg.cond(np.diag(inv.astype(np.float64)) @ dense)
    assert np.linalg.norm(x - want) <= 1e-5 * cond * np.linalg.norm(want)
    true = np.linalg.norm(b - dense @ x)
    assert abs(res - true) <= 1e-4 * true + 1e-6 * np.linalg.norm(b)
    # the plain loop on the badly scaled rows needs more Arnoldi steps
    _, info_p, _, its_p = orc.csr_gmres(A.data, A.indices, A.indptr, b, rtol=1e-5, restart=20,
                                        maxiter=400)
    assert info_p != 0 or its_p > its


def test_gmres_jacobi_status_rules():
    A = np.array([[4.0, 1.0], [1.0, 3.0]], np.float32)
    b = np.array([1.0, 2.0], np.float32)
    # ||M r|| <= FLT_EPSILON while ||r|| > tol: -1 before any step
    for inv in (np.zeros(2, np.float32), np.full(2, 1e-30, np.float32)):
        x, info, res, its = orc.csr_gmres_jacobi(*_csr(A), b, inv, rtol=1e-6)
        assert (info, its) == (-1, 0) and res == np.float32(np.linalg.norm(b))
    inv = np.array([0.25, 1.0 / 3.0], np.float32)
    x, info, res, its = orc.csr_gmres_jacobi(*_csr(A), np.zeros(2, np.float32), inv)
    assert (info, its, res) == (0, 0, 0.0)
    x, info, res, its = orc.csr_gmres_jacobi(*_csr(A), b, inv, maxiter=0)
    assert (info, its) == (1, 0) and res == np.float32(np.linalg.norm(b))
    bad = b.copy()
    bad[1] = np.nan
    _, info, res, its = orc.csr_gmres_jacobi(*_csr(A), bad, inv)
    assert (info, its) == (-3, 0) and np.isinf(res)
