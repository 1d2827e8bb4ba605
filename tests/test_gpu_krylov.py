"""HIP BiCGSTAB and MINRES (msx_csr_bicgstab, msx_csr_minres) against the
oracle through the C ABI, and through ``linalg.bicgstab`` / ``linalg.minres``.

The device loops follow the reference's arithmetic (float SpMV from zero,
double dot products and scalars, vector updates rounded once) but add their
dot products per workgroup, so the rounding of the double sums differs from
the sequential loop.  The bar:

- status equal to the oracle's, iteration count within two (a different
  rounding of a double sum can move the crossing of the tolerance);
- x solves the system as well as the oracle's: error against the float64
  dense solution within rtol * cond, true residual under the tolerance,
  reported residual equal to the true one to float32 rounding;
- the status cases (zero right-hand side, exact x0, maxiter 0 and short
  budgets, non-finite input, breakdown) give the oracle's status,
  iterations and residual;
- a solve is reproducible (two runs give the same bits), on every SpMV route
  (row blocks, LDS panels, no plan);
- the reference's own GPU test systems (tests/test_linalg_bicgstab.py:306-333,
  tests/test_linalg_minres.py:57-93).
"""

from __future__ import annotations

import numpy as np
import pytest
import scipy.sparse as sp
import torch

import _capi
from oracle import oracle as orc
from test_oracle_krylov import INDEF, NONSYM, convection_2d, laplacian_2d

pytestmark = pytest.mark.gpu

DEV = "cuda"


def convection_3d(g, wind=0.3):
    one = sp.diags([-1 - wind, 2, -1 + wind], [-1, 0, 1], shape=(g, g))
    eye = sp.identity(g)
    A = (sp.kron(sp.kron(one, eye), eye) + sp.kron(sp.kron(eye, one), eye)
         + sp.kron(sp.kron(eye, eye), one)).tocsr()
    A.sort_indices()
    return A.astype(np.float32)


def _args(A, index_dtype=np.int32):
    return (A.data.astype(np.float32), A.indices.astype(index_dtype),
            A.indptr.astype(index_dtype))


def _gpu(kind, A, b, index_dtype=np.int32, slice_mode=None, plan=True, x0=None, **kw):
    d, i, p = (torch.from_numpy(np.ascontiguousarray(a)).to(DEV) for a in _args(A, index_dtype))
    pl = _capi.Plan(p, A.shape[0], d.numel(), data=d, indices=i, n_cols=A.shape[1],
                    slice_mode=slice_mode) if plan else None
    out = _capi.krylov(kind, d, i, p, torch.from_numpy(b).to(DEV),
                       None if x0 is None else torch.from_numpy(x0).to(DEV), plan=pl, **kw)
    torch.cuda.synchronize()
    info = pl.info() if pl else None
    return (out[0].cpu().numpy(),) + tuple(out[1:]) + ((info.n_panels if info else 0),)


def _oracle(kind, A, b, index_dtype=np.int32, **kw):
    f = orc.csr_bicgstab if kind == "bicgstab" else orc.csr_minres
    return f(*_args(A, index_dtype), b, **kw)


def _solution_checks(kind, A, b, x, res, rtol, shift=0.0):
    A64 = A.astype(np.float64).toarray() - shift * np.eye(A.shape[0])
    exact = np.linalg.solve(A64, b.astype(np.float64))
    cond = np.linalg.cond(A64)
    assert np.linalg.norm(x - exact) <= 4 * cond * rtol * np.linalg.norm(exact)
    true_res = np.linalg.norm(b.astype(np.float64) - A64 @ x.astype(np.float64))
    assert res <= rtol * np.linalg.norm(b) * (1 + 1e-5), (kind, res)
    assert abs(true_res - res) <= 1e-5 * np.linalg.norm(b) + 1e-3 * res


@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_bicgstab_matches_oracle(index_dtype):
    A = convection_2d(32)
    b = np.random.default_rng(4).uniform(-1, 1, A.shape[0]).astype(np.float32)
    rtol = 1e-4
    print(f"bicgstab convection 32^2 {np.dtype(index_dtype).name}", flush=True)
    x, info, res, its, _ = _gpu("bicgstab", A, b, index_dtype, rtol=rtol)
    wx, winfo, wres, wits = _oracle("bicgstab", A, b, index_dtype, rtol=rtol)
    assert info == winfo == 0 and abs(its - wits) <= 2, (its, wits)
    _solution_checks("bicgstab", A, b, x, res, rtol)


@pytest.mark.parametrize("shift", [0.0, 1.3])
def test_minres_matches_oracle(shift):
    A = laplacian_2d(24)
    b = np.random.default_rng(8).uniform(-1, 1, A.shape[0]).astype(np.float32)
    rtol = 1e-4
    print(f"minres laplacian 24^2 shift={shift}", flush=True)
    x, info, res, its, _ = _gpu("minres", A, b, rtol=rtol, shift=shift)
    wx, winfo, wres, wits = _oracle("minres", A, b, rtol=rtol, shift=shift)
    assert info == winfo == 0 and abs(its - wits) <= 2, (its, wits)
    _solution_checks("minres", A, b, x, res, rtol, shift=shift)


@pytest.mark.parametrize("mode", ["blocks", "panels", "none"])
def test_every_spmv_route_and_reproducible(mode):
    A = convection_3d(40)
    n = A.shape[0]
    b = np.random.default_rng(9).uniform(-1, 1, n).astype(np.float32)
    kw = {"plan": mode != "none",
          "slice_mode": {"blocks": _capi.SLICE_OFF, "panels": _capi.SLICE_PANELS,
                         "none": None}[mode]}
    for kind in ("bicgstab", "minres"):
        M = A if kind == "bicgstab" else laplacian_2d(200)
        bb = b if kind == "bicgstab" else np.random.default_rng(3).uniform(
            -1, 1, M.shape[0]).astype(np.float32)
        print(f"{kind} route={mode} n={M.shape[0]}", flush=True)
        x1, info1, res1, its1, panels = _gpu(kind, M, bb, rtol=1e-4, **kw)
        x2, info2, res2, its2, _ = _gpu(kind, M, bb, rtol=1e-4, **kw)
        if mode == "panels":
            assert panels > 0
        assert (info1, its1) == (info2, its2) and res1 == res2 and x1.tobytes() == x2.tobytes()
        wx, winfo, wres, wits = _oracle(kind, M, bb, rtol=1e-4)
        assert info1 == winfo == 0 and abs(its1 - wits) <= max(2, wits // 50), (its1, wits)
        ref = np.linalg.norm(wx.astype(np.float64))
        assert np.linalg.norm(x1.astype(np.float64) - wx) <= 1e-2 * ref


def test_status_cases_match_oracle():
    A, S = sp.csr_matrix(NONSYM), sp.csr_matrix(INDEF)
    bad = np.ones(4, np.float32)
    bad[2] = np.nan
    exact = np.linalg.solve(NONSYM, np.arange(1, 5, dtype=np.float32)).astype(np.float32)
    bx = (NONSYM.astype(np.float64) @ exact).astype(np.float32)
    cases = [(np.zeros(4, np.float32), {}), (np.ones(4, np.float32), {"maxiter": 0}),
             (np.ones(4, np.float32), {"maxiter": 1, "rtol": 1e-9}), (bad, {})]
    for kind, M in (("bicgstab", A), ("minres", S)):
        for b, kw in cases:
            x, info, res, its, _ = _gpu(kind, M, b, **kw)
            wx, winfo, wres, wits = _oracle(kind, M, b, **kw)
            print(f"{kind} status case {kw}: gpu {info, its, res} oracle {winfo, wits, wres}",
                  flush=True)
            assert (info, its) == (winfo, wits)
            assert np.isnan(res) == np.isnan(wres)
            if not np.isnan(wres):
                assert abs(res - wres) <= 1e-6 * max(1.0, abs(wres))
    x, info, res, its, _ = _gpu("bicgstab", A, bx, x0=exact, rtol=1e-7, atol=1e-7)
    assert (info, its) == (0, 0) and x.tobytes() == exact.tobytes()
    zero = sp.csr_matrix((np.zeros(3, np.float32), np.arange(3), np.arange(4)), shape=(3, 3))
    b1 = np.array([1.0, 0.0, 0.0], np.float32)
    got = _gpu("bicgstab", zero, b1, maxiter=8)
    want = _oracle("bicgstab", zero, b1, maxiter=8)
    assert got[1] == want[1] < 0 and got[3] == want[3]


def test_hand_computed_and_closed_forms():
    x, info, res, its, _ = _gpu("bicgstab", sp.csr_matrix(np.diag([1.0, 2.0]).astype(np.float32)),
                                np.ones(2, np.float32), rtol=1e-5)
    assert (info, its) == (0, 2)
    np.testing.assert_allclose(x, [1.0, 0.5], rtol=1e-6, atol=1e-7)
    rng = np.random.default_rng(3)
    n, eigs = 40, [2.0, 5.0, -1.0]
    diag = np.array([eigs[j % 3] for j in range(n)])
    Q, _ = np.linalg.qr(rng.standard_normal((n, n)))
    dense = ((Q * diag) @ Q.T).astype(np.float32)
    dense = (dense + dense.T) / 2
    b = rng.uniform(-1, 1, n).astype(np.float32)
    x, info, res, its, _ = _gpu("minres", sp.csr_matrix(dense), b, rtol=1e-4)
    assert (info, its) == (0, 3)


def test_api_on_gpu_reference_systems(gpu):
    """The reference's GPU tests (test_linalg_bicgstab.py:306-333,
    test_linalg_minres.py:57-93) through linalg on the device."""
    ms = gpu
    from mlx_sparse import linalg

    def csr(dense):
        A = sp.csr_matrix(dense.astype(np.float32))
        return ms.csr_array((A.data, A.indices.astype(np.int32), A.indptr.astype(np.int32)),
                            shape=dense.shape, canonical=True)

    b = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    x, info = linalg.bicgstab(csr(NONSYM), b, rtol=1e-6, atol=1e-7, maxiter=80)
    assert info == 0 and x.device.type == "cuda"
    xn = x.cpu().numpy().astype(np.float64)
    assert np.linalg.norm(NONSYM @ xn - b) / max(np.linalg.norm(b), 1.0) < 2e-6
    bi = np.array([1.0, -2.0, 0.5, 3.0], np.float32)
    x, info = linalg.minres(csr(INDEF), bi, rtol=1e-6, atol=1e-7, maxiter=64)
    assert info == 0
    np.testing.assert_allclose(x.cpu().numpy(), np.linalg.solve(INDEF, bi), rtol=5e-5, atol=5e-5)
    x, info = linalg.minres(csr(np.diag([0.0, 2.0, 3.0, -4.0])),
                            np.array([0.0, 4.0, -3.0, 8.0], np.float32), rtol=1e-7, atol=1e-7,
                            maxiter=32, return_info=True)
    assert info.status == 0 and info.solver == "minres"


def test_full_size_minres_and_bicgstab(gpu):
    """Both loops at the SpMM benchmark's size (n = 128^3) on the device
    with the matrix's cached plan, against the oracle: MINRES on the 3D
    Poisson matrix with shift -1 (A + I), BiCGSTAB on a nonsymmetric
    convection-diffusion variant of it (x-direction off-diagonals -1.3 and
    -0.7, diagonal 8).  In float32 the reference's loops stagnate near a
    relative residual of 1e-3 on the plain Poisson matrix (MINRES) or break
    down (BiCGSTAB, rho = 0 against r_hat = b), so these are the systems
    both converge on."""
    ms = gpu
    from mlx_sparse import linalg, synthetic

    m = synthetic.poisson_3d(128)
    n = m.shape[0]
    rows = np.repeat(np.arange(n), np.diff(m.indptr))
    cols = m.indices.astype(np.int64)
    conv = m.data.copy()
    conv[cols == rows + 1] = -0.7
    conv[cols == rows - 1] = -1.3
    conv[cols == rows] = 8.0
    b_np = synthetic.uniform(n, -1.0, 1.0, seed=7)
    b = torch.from_numpy(b_np).to(DEV)
    for name, data, kw in (("minres", m.data, {"shift": -1.0}), ("bicgstab", conv, {})):
        A = ms.csr_array((data, m.indices, m.indptr), shape=m.shape, canonical=True)
        solver = getattr(linalg, name)
        x, info = solver(A, b, rtol=1e-5, maxiter=500, return_info=True, **kw)
        wx, winfo, wres, wits = _oracle(name, sp.csr_matrix((data, m.indices, m.indptr),
                                                            shape=m.shape), b_np, rtol=1e-5,
                                        maxiter=500, **kw)
        print(f"{name}: gpu status {info.status} iterations {info.iterations} residual "
              f"{info.residual_norm:.5g}; oracle {winfo} {wits} {wres:.5g}", flush=True)
        assert info.status == winfo == 0 and abs(info.iterations - wits) <= 2
        assert info.residual_norm <= 1e-5 * np.linalg.norm(b_np) * (1 + 1e-5)
        ref = np.linalg.norm(wx.astype(np.float64))
        assert np.linalg.norm(x.cpu().numpy().astype(np.float64) - wx) <= 1e-4 * ref


# -- BiCGSTAB with a Jacobi preconditioner (msx_csr_bicgstab_jacobi) ------------------

def _scaled_convection(g, seed=9):
    """convection_2d(g) with rows scaled by 10^U[-2, 2]: the plain loop
    struggles, the Jacobi loop does not."""
    A0 = convection_2d(g)
    rng = np.random.default_rng(seed)
    scale = np.float32(10.0) ** rng.uniform(-2, 2, A0.shape[0]).astype(np.float32)
    A = (sp.diags(scale) @ A0).tocsr().astype(np.float32)
    A.sort_indices()
    b = (scale * rng.uniform(-1, 1, A.shape[0])).astype(np.float32)
    return A, b, (1.0 / A.diagonal()).astype(np.float32)


def _gpu_jacobi(A, b, inv, index_dtype=np.int32, slice_mode=None, plan=True, x0=None, **kw):
    d, i, p = (torch.from_numpy(np.ascontiguousarray(a)).to(DEV) for a in _args(A, index_dtype))
    pl = _capi.Plan(p, A.shape[0], d.numel(), data=d, indices=i, n_cols=A.shape[1],
                    slice_mode=slice_mode) if plan else None
    out = _capi.krylov("bicgstab", d, i, p, torch.from_numpy(b).to(DEV),
                       None if x0 is None else torch.from_numpy(x0).to(DEV), plan=pl,
                       inv_diag=torch.from_numpy(inv).to(DEV), **kw)
    torch.cuda.synchronize()
    return (out[0].cpu().numpy(),) + tuple(out[1:])


@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_bicgstab_jacobi_matches_oracle(index_dtype):
    """Status equal to the oracle's, iterations within two, x solving the
    system, the reported residual the true one - on the row-scaled system
    and on the plain convection system."""
    # float32 BiCGSTAB stops with -1 once r turns orthogonal to r_hat (the
    # reference's relative rho test), on either side depending on rounding:
    # tolerances where the oracle converges with margin (it still converges
    # at a third of them)
    for g, scaled, rtol in ((48, True, 1e-4), (32, False, 1e-5)):
        if scaled:
            A, b, inv = _scaled_convection(g, seed=3)
        else:
            A = convection_2d(g)
            b = np.random.default_rng(4).uniform(-1, 1, A.shape[0]).astype(np.float32)
            inv = (1.0 / A.diagonal()).astype(np.float32)
        print(f"bicgstab jacobi g={g} scaled={scaled} {np.dtype(index_dtype).name}", flush=True)
        x, info, res, its = _gpu_jacobi(A, b, inv, index_dtype, rtol=rtol, maxiter=600)
        wx, winfo, wres, wits = orc.csr_bicgstab_jacobi(*_args(A, index_dtype), b, inv,
                                                        rtol=rtol, maxiter=600)
        assert info == winfo == 0 and abs(its - wits) <= 2, (its, wits)
        dense = A.toarray().astype(np.float64)
        want = np.linalg.solve(dense, b.astype(np.float64))
        cond = np.linalg.cond(np.diag(inv.astype(np.float64)) @ dense)
        assert np.linalg.norm(x - want) <= 4 * rtol * cond * np.linalg.norm(want)
        true_res = np.linalg.norm(b.astype(np.float64) - dense @ x.astype(np.float64))
        assert res <= rtol * np.linalg.norm(b) * (1 + 1e-5)
        assert abs(true_res - res) <= 1e-5 * np.linalg.norm(b) + 1e-3 * res


@pytest.mark.parametrize("mode", ["blocks", "panels", "none"])
def test_bicgstab_jacobi_routes_and_reproducible(mode):
    A, b, inv = _scaled_convection(96, seed=2)
    kw = {"plan": mode != "none",
          "slice_mode": {"blocks": _capi.SLICE_OFF, "panels": _capi.SLICE_PANELS,
                         "none": None}[mode]}
    print(f"bicgstab jacobi route={mode} n={A.shape[0]}", flush=True)
    r1 = _gpu_jacobi(A, b, inv, rtol=1e-4, maxiter=2000, **kw)
    r2 = _gpu_jacobi(A, b, inv, rtol=1e-4, maxiter=2000, **kw)
    assert r1[1:] == r2[1:] and r1[0].tobytes() == r2[0].tobytes()
    wx, winfo, wres, wits = orc.csr_bicgstab_jacobi(*_args(A), b, inv, rtol=1e-4, maxiter=2000)
    # BiCGSTAB's residual is not monotone: on this row-scaled system another
    # rounding of the double dot products moves the tolerance crossing by a
    # few percent of the iterations
    assert r1[1] == winfo == 0 and abs(r1[3] - wits) <= max(2, wits // 20), (r1[3], wits)
    assert np.linalg.norm(r1[0].astype(np.float64) - wx) <= 1e-2 * np.linalg.norm(wx)


def test_bicgstab_jacobi_status_cases_match_oracle():
    """The edge cases where the Jacobi loop differs from the plain one: a
    non-finite b (status -3, residual +inf), a non-finite inverse diagonal
    entry (-3 in the first iteration), plus a zero right-hand side, an exact
    x0, maxiter 0 and 1."""
    A = sp.csr_matrix(NONSYM)
    inv = (1.0 / np.diag(NONSYM)).astype(np.float32)
    b = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    bad_b = b.copy()
    bad_b[2] = np.nan
    bad_inv = inv.copy()
    bad_inv[1] = np.inf
    exact = np.linalg.solve(NONSYM, b).astype(np.float32)
    bx = (NONSYM.astype(np.float64) @ exact).astype(np.float32)
    cases = [(np.zeros(4, np.float32), inv, None, {}), (b, inv, None, {"maxiter": 0}),
             (b, inv, None, {"maxiter": 1, "rtol": 1e-9}), (bad_b, inv, None, {}),
             (b, bad_inv, None, {}), (bx, inv, exact, {"rtol": 1e-3}),
             (b, inv, None, {"rtol": 1e-4, "atol": 1e-7, "maxiter": 80})]
    for rhs, iv, x0, kw in cases:
        x, info, res, its = _gpu_jacobi(A, rhs, iv, x0=x0, **kw)
        wx, winfo, wres, wits = orc.csr_bicgstab_jacobi(*_args(A), rhs, iv, x0, **kw)
        print(f"jacobi status case {kw}: gpu {info, its, res} oracle {winfo, wits, wres}",
              flush=True)
        assert (info, its) == (winfo, wits)
        assert np.isinf(res) == np.isinf(wres) and np.isnan(res) == np.isnan(wres)
        if np.isfinite(wres):
            assert abs(res - wres) <= 1e-6 * max(1.0, abs(wres))


def test_bicgstab_jacobi_api_on_gpu(gpu):
    """linalg.bicgstab with M = preconditioners.jacobi(A) on the device: the
    reference's GPU test (test_linalg_bicgstab.py:313-333) and its bounds."""
    ms = gpu
    from mlx_sparse import linalg
    from mlx_sparse.linalg import preconditioners

    A = sp.csr_matrix(NONSYM)
    csr = ms.csr_array((A.data, A.indices.astype(np.int32), A.indptr.astype(np.int32)),
                       shape=NONSYM.shape, canonical=True)
    b = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    x, info = linalg.bicgstab(csr, b, M=preconditioners.jacobi(csr), rtol=1e-4, atol=1e-7,
                              maxiter=80, return_info=True)
    assert info.status == 0 and info.preconditioner == "jacobi" and x.device.type == "cuda"
    xn = x.cpu().numpy().astype(np.float64)
    assert np.linalg.norm(NONSYM @ xn - b) / max(np.linalg.norm(b), 1.0) < 2e-5


# -- MINRES with a Jacobi preconditioner (msx_csr_minres_jacobi) ----------------------

def _scaled_laplacian(g, seed=6):
    """S L S for the 2D Laplacian L and S = diag(10^U[-1/2, 1/2]): symmetric
    positive definite and badly scaled.  (Scaled over two decades the
    float32 loop stagnates above 1e-5 relative residual, in the oracle as
    on the device.)"""
    A = laplacian_2d(g)
    rng = np.random.default_rng(seed)
    s = (10.0 ** rng.uniform(-0.5, 0.5, A.shape[0])).astype(np.float32)
    As = (sp.diags(s) @ A @ sp.diags(s)).tocsr().astype(np.float32)
    As.sort_indices()
    b = rng.uniform(-1, 1, A.shape[0]).astype(np.float32)
    return As, b, (1.0 / As.diagonal()).astype(np.float32)


def _gpu_minres_jacobi(A, b, inv, slice_mode=None, plan=True, x0=None, **kw):
    d, i, p = (torch.from_numpy(np.ascontiguousarray(a)).to(DEV) for a in _args(A))
    pl = _capi.Plan(p, A.shape[0], d.numel(), data=d, indices=i, n_cols=A.shape[1],
                    slice_mode=slice_mode) if plan else None
    out = _capi.krylov("minres", d, i, p, torch.from_numpy(b).to(DEV),
                       None if x0 is None else torch.from_numpy(x0).to(DEV), plan=pl,
                       inv_diag=torch.from_numpy(inv).to(DEV), **kw)
    torch.cuda.synchronize()
    return (out[0].cpu().numpy(),) + tuple(out[1:])


@pytest.mark.parametrize("shift", [0.0, -0.3, 1.3])
def test_minres_jacobi_matches_oracle(shift):
    A, b, inv = _scaled_laplacian(32)
    rtol = 1e-4  # the oracle converges at a tenth of it too
    print(f"minres jacobi scaled laplacian 32^2 shift={shift}", flush=True)
    x, info, res, its = _gpu_minres_jacobi(A, b, inv, rtol=rtol, shift=shift, maxiter=3000)
    wx, winfo, wres, wits = orc.csr_minres_jacobi(*_args(A), b, inv, rtol=rtol, shift=shift,
                                                  maxiter=3000)
    assert info == winfo == 0 and abs(its - wits) <= max(2, wits // 50), (its, wits)
    dense = A.toarray().astype(np.float64) - shift * np.eye(A.shape[0])
    want = np.linalg.solve(dense, b.astype(np.float64))
    cond = np.linalg.cond(dense)
    assert np.linalg.norm(x - want) <= 4 * rtol * cond * np.linalg.norm(want)
    true_res = np.linalg.norm(b.astype(np.float64) - dense @ x.astype(np.float64))
    assert res <= rtol * np.linalg.norm(b) * (1 + 1e-5)
    assert abs(true_res - res) <= 1e-5 * np.linalg.norm(b) + 1e-3 * res


@pytest.mark.parametrize("mode", ["blocks", "panels", "none"])
def test_minres_jacobi_routes_and_reproducible(mode):
    A, b, inv = _scaled_laplacian(100, seed=2)
    kw = {"plan": mode != "none",
          "slice_mode": {"blocks": _capi.SLICE_OFF, "panels": _capi.SLICE_PANELS,
                         "none": None}[mode]}
    print(f"minres jacobi route={mode} n={A.shape[0]}", flush=True)
    r1 = _gpu_minres_jacobi(A, b, inv, rtol=1e-4, maxiter=5000, **kw)
    r2 = _gpu_minres_jacobi(A, b, inv, rtol=1e-4, maxiter=5000, **kw)
    assert r1[1:] == r2[1:] and r1[0].tobytes() == r2[0].tobytes()
    wx, winfo, wres, wits = orc.csr_minres_jacobi(*_args(A), b, inv, rtol=1e-4, maxiter=5000)
    assert r1[1] == winfo == 0 and abs(r1[3] - wits) <= max(2, wits // 50), (r1[3], wits)
    assert np.linalg.norm(r1[0].astype(np.float64) - wx) <= 1e-2 * np.linalg.norm(wx)


def test_minres_jacobi_status_cases_match_oracle():
    """-2 for an inverse diagonal entry that is not > 0 (negative, zero, NaN)
    or a non-finite preconditioned product (an infinite entry); a zero
    right-hand side; maxiter 0 and 1; a non-finite b."""
    S = sp.csr_matrix(INDEF)
    b = np.array([1.0, -2.0, 0.5, 3.0], np.float32)
    good = np.full(4, 0.5, np.float32)
    bad_b = b.copy()
    bad_b[0] = np.inf
    cases = [(b, good, {}), (np.zeros(4, np.float32), good, {}), (b, good, {"maxiter": 0}),
             (b, good, {"maxiter": 1, "rtol": 1e-9}), (bad_b, good, {})]
    for v in (-1.0, 0.0, np.nan, np.inf):
        inv = good.copy()
        inv[1] = v
        cases.append((b, inv, {}))
    for rhs, iv, kw in cases:
        x, info, res, its = _gpu_minres_jacobi(S, rhs, iv, **kw)
        wx, winfo, wres, wits = orc.csr_minres_jacobi(*_args(S), rhs, iv, **kw)
        print(f"minres jacobi status case {kw} inv={iv}: gpu {info, its, res} "
              f"oracle {winfo, wits, wres}", flush=True)
        assert (info, its) == (winfo, wits)
        assert np.isnan(res) == np.isnan(wres) and np.isinf(res) == np.isinf(wres)
        if np.isfinite(wres):
            assert abs(res - wres) <= 1e-6 * max(1.0, abs(wres))


def test_minres_jacobi_api_on_gpu(gpu):
    """linalg.minres with a Jacobi preconditioner on the device: the
    reference's diagonal-preconditioner test and its bounds
    (test_linalg_minres.py:141-179)."""
    ms = gpu
    from mlx_sparse import linalg
    from mlx_sparse.linalg import preconditioners

    dense = np.array([[2.0, 3.0, 0.0], [3.0, 2.0, 0.5], [0.0, 0.5, 4.0]], np.float32)
    A = sp.csr_matrix(dense)
    csr = ms.csr_array((A.data, A.indices.astype(np.int32), A.indptr.astype(np.int32)),
                       shape=dense.shape, canonical=True)
    b = np.array([1.0, -2.0, 0.5], np.float32)
    x, info = linalg.minres(csr, b, M=preconditioners.jacobi(csr, check=True), rtol=1e-6,
                            atol=1e-7, maxiter=64, return_info=True)
    assert info.status == 0 and x.device.type == "cuda"
    xn = x.cpu().numpy()
    np.testing.assert_allclose(xn, np.linalg.solve(dense, b), rtol=5e-5, atol=5e-5)
    assert np.linalg.norm(dense.astype(np.float64) @ xn - b) / np.linalg.norm(b) < 2e-6


def test_full_size_jacobi_solvers(gpu):
    """The four Jacobi-preconditioned loops at n = 128^3 on the device with
    the matrix's cached plan, against the oracle, on rows scaled by
    10^U[-1, 1] (which the inverse diagonal undoes): BiCGSTAB and GMRES(20)
    on the convection-diffusion variant scaled by rows, CG and MINRES on the
    Poisson matrix (plus the identity for MINRES) scaled on both sides, so
    it stays symmetric.  Status equal, iterations within two (GMRES: one
    cycle), the reported residual under the tolerance, the true residual
    of x as small as that of the oracle's x, x within 1e-3 of the
    oracle's."""
    ms = gpu
    from mlx_sparse import linalg, synthetic
    from mlx_sparse.linalg import preconditioners

    m = synthetic.poisson_3d(128)
    n = m.shape[0]
    rows = np.repeat(np.arange(n), np.diff(m.indptr))
    cols = m.indices.astype(np.int64)
    conv = m.data.copy()
    conv[cols == rows + 1] = -0.7
    conv[cols == rows - 1] = -1.3
    conv[cols == rows] = 8.0
    s = (10.0 ** np.random.default_rng(11).uniform(-1, 1, n)).astype(np.float32)
    conv_s = (conv * s[rows]).astype(np.float32)
    pois_s = (m.data * s[rows] * s[cols]).astype(np.float32)
    shifted = m.data.copy()
    shifted[cols == rows] += 1.0
    shifted_s = (shifted * s[rows] * s[cols]).astype(np.float32)
    b_np = synthetic.uniform(n, -1.0, 1.0, seed=7)
    b = torch.from_numpy(b_np).to(DEV)
    cases = (("bicgstab", conv_s, orc.csr_bicgstab_jacobi, {"maxiter": 500}, 2),
             ("gmres", conv_s, orc.csr_gmres_jacobi, {"restart": 20, "maxiter": 400}, 20),
             ("cg", pois_s, orc.csr_pcg_jacobi, {"maxiter": 2000}, 2),
             ("minres", shifted_s, orc.csr_minres_jacobi, {"maxiter": 500}, 2))
    for name, data, oracle_fn, kw, slack in cases:
        A = ms.csr_array((data, m.indices, m.indptr), shape=m.shape, canonical=True)
        inv = (1.0 / data[cols == rows]).astype(np.float32)
        x, info = getattr(linalg, name)(A, b, M=preconditioners.jacobi(A), rtol=1e-5,
                                        return_info=True, **kw)
        wx, winfo, wres, wits = oracle_fn(data, m.indices, m.indptr, b_np, inv, rtol=1e-5, **kw)
        print(f"{name} jacobi: gpu status {info.status} iterations {info.iterations} residual "
              f"{info.residual_norm:.5g}; oracle {winfo} {wits} {wres:.5g}", flush=True)
        assert info.status == winfo == 0 and abs(info.iterations - wits) <= slack
        assert info.preconditioner == "jacobi"
        assert info.residual_norm <= 1e-5 * np.linalg.norm(b_np) * (1 + 1e-5)
        xn = x.cpu().numpy().astype(np.float64)
        A64 = sp.csr_matrix((data.astype(np.float64), m.indices, m.indptr), shape=m.shape)
        # The recurrence residual drifts from the true one in float32 (CG over
        # hundreds of steps on a badly scaled system most): the oracle's x
        # carries the same drift, so the true residuals are compared.
        true_res = np.linalg.norm(b_np - A64 @ xn)
        true_orc = np.linalg.norm(b_np - A64 @ wx.astype(np.float64))
        print(f"  true residual {true_res:.5g}; oracle's x {true_orc:.5g}", flush=True)
        assert true_res <= 1.5 * true_orc + 1e-5 * np.linalg.norm(b_np)
        ref = np.linalg.norm(wx.astype(np.float64))
        print(f"  |x - x_oracle| / |x_oracle| = {np.linalg.norm(xn - wx) / ref:.3g}", flush=True)
        assert np.linalg.norm(xn - wx) <= 1e-3 * ref
