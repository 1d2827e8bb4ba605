"""HIP restarted GMRES (msx_csr_gmres) against the oracle through the C ABI,
and through ``linalg.gmres``.

The device Arnoldi follows the reference's CPU arithmetic (float SpMV from
zero, two sweeps of modified Gram-Schmidt with double sums of float
products, float subtractions, norm_float) with two differences: each dot
product is added per workgroup, and the projections are taken in pairs per
pass over w, the second coefficient of a pair as d_b - c_a (q_a.q_b) from
sums taken before the first projection (equal to the sequential one in
exact arithmetic), so the rounding differs from the sequential loop; the
small least-squares problem and the restart logic run on the host exactly
as in the oracle.  The bar:

- status equal to the oracle's; iterations equal on cases whose stopping
  cycle is not at the tolerance's edge, else within one cycle;
- x solves the system as well as the oracle's: error against the float64
  dense solution within rtol * cond, reported residual equal to the true
  residual of the returned x to float32 rounding, and x within 1e-4 of the
  oracle's x;
- the status cases (zero right-hand side, exact x0, maxiter 0 and short
  budgets, non-finite input or value, an Arnoldi breakdown) give the
  oracle's status, iterations and residual; the Hilbert 5x5 case, which the
  budget ends at float32 rounding, meets the reference's own residual bound;
- a solve is reproducible (two runs give the same bits), on every SpMV route
  (row blocks, LDS panels, no plan);
- the reference's own GPU-reachable test systems
  (tests/test_linalg_pathological.py:499-659, test_linalg_native.py:105-115);
- n = 128^3 against the oracle for three restart cycles.
"""

from __future__ import annotations

import numpy as np
import pytest
import scipy.sparse as sp
import torch

import _capi
from oracle import oracle as orc
from test_gpu_krylov import convection_3d
from test_oracle_gmres import _csr, _random_nonsym

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _args(A, index_dtype=np.int32):
    return (A.data.astype(np.float32), A.indices.astype(index_dtype),
            A.indptr.astype(index_dtype))


def _gpu(A, b, index_dtype=np.int32, slice_mode=None, plan=True, x0=None, **kw):
    d, i, p = (torch.from_numpy(np.ascontiguousarray(a)).to(DEV) for a in _args(A, index_dtype))
    pl = _capi.Plan(p, A.shape[0], d.numel(), data=d, indices=i, n_cols=A.shape[1],
                    slice_mode=slice_mode) if plan else None
    out = _capi.gmres(d, i, p, torch.from_numpy(b).to(DEV),
                      None if x0 is None else torch.from_numpy(x0).to(DEV), plan=pl, **kw)
    torch.cuda.synchronize()
    info = pl.info() if pl else None
    return (out[0].cpu().numpy(),) + tuple(out[1:]) + ((info.n_panels if info else 0),)


def _solution_checks(A, b, x, res, rtol, wx=None):
    A64 = A.astype(np.float64).toarray()
    exact = np.linalg.solve(A64, b.astype(np.float64))
    cond = np.linalg.cond(A64)
    assert np.linalg.norm(x - exact) <= 4 * cond * rtol * np.linalg.norm(exact)
    true_res = np.linalg.norm(b.astype(np.float64) - A64 @ x.astype(np.float64))
    assert res <= rtol * np.linalg.norm(b) * (1 + 1e-5), res
    assert abs(true_res - res) <= 1e-5 * np.linalg.norm(b) + 1e-3 * res
    if wx is not None:
        assert np.linalg.norm(x - wx) <= 1e-4 * np.linalg.norm(wx) + 4 * cond * rtol * \
            np.linalg.norm(exact)


@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
@pytest.mark.parametrize("restart", [1, 5, 20, 64])
def test_gmres_matches_oracle(index_dtype, restart):
    A = _random_nonsym(1200, seed=restart, density=0.005, shift=0.5)
    b = np.random.default_rng(restart).uniform(-1, 1, A.shape[0]).astype(np.float32)
    rtol = 1e-5
    print(f"gmres random n=1200 restart={restart} {np.dtype(index_dtype).name}", flush=True)
    x, info, res, its, _ = _gpu(A, b, index_dtype, rtol=rtol, restart=restart, maxiter=20000)
    wx, winfo, wres, wits = orc.csr_gmres(*_args(A, index_dtype), b, rtol=rtol, restart=restart,
                                          maxiter=20000)
    assert info == winfo == 0 and abs(its - wits) <= restart, (its, wits)
    _solution_checks(A, b, x, res, rtol, wx)


@pytest.mark.parametrize("restart", [4, 30])
def test_gmres_nonsymmetric_convection_matches_oracle(restart):
    A = convection_3d(12, wind=0.6)
    b = np.random.default_rng(2).uniform(-1, 1, A.shape[0]).astype(np.float32)
    print(f"gmres convection 12^3 restart={restart}", flush=True)
    x, info, res, its, _ = _gpu(A, b, rtol=1e-5, restart=restart)
    wx, winfo, wres, wits = orc.csr_gmres(*_args(A), b, rtol=1e-5, restart=restart)
    assert info == winfo == 0 and abs(its - wits) <= restart, (its, wits)
    _solution_checks(A, b, x, res, 1e-5, wx)


@pytest.mark.parametrize("case", ["zero_rhs", "exact", "nan_b", "inf_x0", "nan_value",
                                  "maxiter0", "short", "breakdown", "hilbert"])
def test_gmres_status_cases_equal_oracle(case):
    dense = np.diag([2.0, 3.0, 4.0, 5.0, 6.0, 7.0]).astype(np.float32)
    dense[0, 5] = 0.5
    b = np.ones(6, np.float32)
    x0 = None
    kw = {}
    if case == "zero_rhs":
        b = np.zeros(6, np.float32)
    elif case == "exact":
        x0 = np.linspace(-1.0, 1.0, 6, dtype=np.float32)
        b = (dense.astype(np.float64) @ x0.astype(np.float64)).astype(np.float32)
        kw = {"atol": 1e-5}
    elif case == "nan_b":
        b[2] = np.nan
    elif case == "inf_x0":
        x0 = np.zeros(6, np.float32)
        x0[1] = np.inf
    elif case == "maxiter0":
        kw = {"maxiter": 0}
    elif case == "short":
        kw = {"maxiter": 3, "restart": 2, "rtol": 1e-9}
    elif case == "breakdown":
        dense = np.diag([1.0, 2.0, 3.0, 4.0, 5.0, 6.0]).astype(np.float32)
        b = np.array([1.0, 0.0, 1.0, 0.0, 1.0, 0.0], np.float32)  # invariant subspace, dim 3
        kw = {"restart": 6, "rtol": 1e-7}
    elif case == "hilbert":
        i = np.arange(5, dtype=np.float32)
        dense = (1.0 / (i[:, None] + i[None, :] + 1.0)).astype(np.float32)
        b = np.linspace(0.25, 1.25, 5, dtype=np.float32)
        kw = {"rtol": 1e-6, "atol": 1e-7, "restart": 5, "maxiter": 64}
    d, ix, ip = _csr(dense)
    if case == "nan_value":
        d = d.copy()
        d[0] = np.nan
    A = sp.csr_matrix((d, ix, ip), shape=dense.shape)
    print(f"gmres status case {case}", flush=True)
    x, info, res, its, _ = _gpu(A, b, x0=x0, **kw)
    wx, winfo, wres, wits = orc.csr_gmres(d, ix, ip, b, x0, **kw)
    assert (info, its) == (winfo, wits), (case, info, its, winfo, wits)
    if np.isnan(wres):
        assert np.isnan(res)
    elif case == "hilbert":
        # cond ~ 5e5, ||x|| ~ 8e3 and the budget ends the solve: the
        # residual is where float rounding leaves it (the device's paired
        # Gram-Schmidt rounds differently from the sequential loop), so the
        # check is the reference's own bound on the returned x
        # (tests/test_linalg_pathological.py:615-643), the reported residual
        # within the float32 rounding of b - A x of the true one, and the
        # error bound of the true residual
        A64 = dense.astype(np.float64)
        x64 = x.astype(np.float64)
        true_res = np.linalg.norm(A64 @ x64 - b)
        assert true_res / max(np.linalg.norm(b), 1.0) < 2e-4
        assert res / max(np.linalg.norm(b), 1.0) < 2e-4
        rounding = 8 * np.finfo(np.float32).eps * np.linalg.norm(np.abs(A64) @ np.abs(x64) + np.abs(b))
        assert abs(true_res - res) <= rounding
        exact = np.linalg.solve(A64, b.astype(np.float64))
        cond = np.linalg.cond(A64)
        assert np.linalg.norm(x - exact) <= cond * true_res / np.linalg.norm(b) * np.linalg.norm(exact)
        return
    else:
        assert res == pytest.approx(wres, rel=1e-5, abs=1e-7)
    finite = np.isfinite(wx)
    np.testing.assert_array_equal(np.isfinite(x), finite)
    np.testing.assert_allclose(x[finite], wx[finite], rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("mode", ["blocks", "panels", "none"])
def test_gmres_every_spmv_route_and_reproducible(mode):
    A = convection_3d(40)
    b = np.random.default_rng(9).uniform(-1, 1, A.shape[0]).astype(np.float32)
    kw = {"plan": mode != "none",
          "slice_mode": {"blocks": _capi.SLICE_OFF, "panels": _capi.SLICE_PANELS,
                         "none": None}[mode]}
    print(f"gmres route={mode} n={A.shape[0]}", flush=True)
    x1, info1, res1, its1, panels = _gpu(A, b, rtol=1e-5, restart=10, **kw)
    x2, info2, res2, its2, _ = _gpu(A, b, rtol=1e-5, restart=10, **kw)
    if mode == "panels":
        assert panels > 0
    assert info1 == 0
    assert (info1, its1) == (info2, its2) and res1 == res2 and x1.tobytes() == x2.tobytes()
    wx, winfo, wres, wits = orc.csr_gmres(*_args(A), b, rtol=1e-5, restart=10)
    assert winfo == 0 and abs(its1 - wits) <= 10
    true_res = np.linalg.norm(b - A.astype(np.float64) @ x1.astype(np.float64))
    assert res1 <= 1e-5 * np.linalg.norm(b) * (1 + 1e-5)
    assert abs(true_res - res1) <= 1e-5 * np.linalg.norm(b) + 1e-3 * res1


def test_linalg_gmres_reference_systems(gpu):
    """The reference's GMRES systems through the drop-in API on the GPU:
    the 2x2 SPD system, the 3x3 that converges on its last restart, the 5x5
    nonsymmetric system against numpy, the Hilbert-like 5x5 whose residual
    stays bounded (tests/test_linalg_pathological.py:499-659)."""
    ms = gpu
    from mlx_sparse import linalg

    def csr(dense):
        d, ix, ip = _csr(dense)
        return ms.csr_array((torch.from_numpy(d), torch.from_numpy(ix), torch.from_numpy(ip)),
                            shape=dense.shape)

    dense = np.array([[4.0, 1.0], [1.0, 3.0]], np.float32)
    x, info = linalg.gmres(csr(dense), np.array([1.0, 2.0], np.float32), rtol=1e-6, atol=1e-7,
                           maxiter=20)
    assert info == 0 and x.device.type == "cuda"
    np.testing.assert_allclose(x.cpu().numpy(), np.linalg.solve(dense, [1.0, 2.0]), rtol=5e-4,
                               atol=5e-4)
    dense = np.array([[4.0, -1.0, 0.25], [0.5, 3.5, -0.75], [0.0, 0.4, 2.75]], np.float32)
    b = np.array([1.0, -2.0, 0.5], np.float32)
    x, info = linalg.gmres(csr(dense), b, rtol=1e-6, atol=1e-7, restart=3, maxiter=3)
    assert info == 0
    np.testing.assert_allclose(x.cpu().numpy(), np.linalg.solve(dense.astype(np.float64), b),
                               rtol=5e-5, atol=5e-5)
    dense = np.array([[5.0, -1.0, 0.5, 0.0, 0.0], [0.2, 4.5, -0.7, 0.4, 0.0],
                      [0.0, -0.3, 5.2, 1.1, 0.2], [0.0, 0.6, -0.2, 4.8, -1.0],
                      [0.1, 0.0, 0.5, -0.4, 3.9]], np.float32)
    b = np.array([1.0, -2.0, 0.5, 3.0, -1.5], np.float32)
    x, info = linalg.gmres(csr(dense), b, rtol=1e-6, atol=1e-7, restart=4, maxiter=40,
                           return_info=True)
    assert info.status == 0 and info.solver == "gmres" and info.restart == 4
    np.testing.assert_allclose(x.cpu().numpy(), np.linalg.solve(dense.astype(np.float64), b),
                               rtol=5e-5, atol=5e-5)
    i = np.arange(5, dtype=np.float32)
    dense = (1.0 / (i[:, None] + i[None, :] + 1.0)).astype(np.float32)
    b = np.linspace(0.25, 1.25, 5, dtype=np.float32)
    x, info = linalg.gmres(csr(dense), b, rtol=1e-6, atol=1e-7, restart=5, maxiter=64)
    rel = np.linalg.norm(dense.astype(np.float64) @ x.cpu().numpy() - b) / np.linalg.norm(b)
    assert info > 0 and np.isfinite(rel) and rel < 2e-4


def test_full_size_gmres_three_cycles(gpu):
    """n = 128^3 (the SpMM benchmark's matrix, with the x-direction
    convection of the full-size BiCGSTAB test): three cycles of 20 Arnoldi
    steps on the device with the matrix's cached plan, against the oracle's
    loop: same status and iterations, residual within 1e-3 and x within
    1e-4."""
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
    A = ms.csr_array((conv, m.indices, m.indptr), shape=m.shape, canonical=True)
    print("gmres 128^3, 3 cycles of 20", flush=True)
    x, info = linalg.gmres(A, torch.from_numpy(b_np).to(DEV), rtol=1e-7, restart=20, maxiter=60,
                           return_info=True)
    wx, winfo, wres, wits = orc.csr_gmres(conv, m.indices, m.indptr, b_np, rtol=1e-7, restart=20,
                                          maxiter=60)
    print(f"gmres 128^3: gpu status {info.status} iterations {info.iterations} residual "
          f"{info.residual_norm:.6g}; oracle {winfo} {wits} {wres:.6g}", flush=True)
    assert (info.status, info.iterations) == (winfo, wits)
    # the residual ends near 1e-7 of ||b||, where the float32 b - A x of
    # either loop rounds: within 1e-3 of each other (the paired Gram-Schmidt
    # passes round differently from the sequential ones)
    assert abs(info.residual_norm - wres) <= 1e-3 * wres
    ref = np.linalg.norm(wx.astype(np.float64))
    assert np.linalg.norm(x.cpu().numpy().astype(np.float64) - wx) <= 1e-4 * ref


# -- GMRES with a Jacobi preconditioner (msx_csr_gmres_jacobi) ----------------------------

def _row_scaled(A0, seed, decades=1.0):
    """A0 with rows scaled by 10^U[-decades, decades] and its inverse
    diagonal: the Jacobi loop undoes the scaling, the plain loop needs many
    more Arnoldi steps."""
    rng = np.random.default_rng(seed)
    s = (10.0 ** rng.uniform(-decades, decades, A0.shape[0])).astype(np.float32)
    A = (sp.diags(s) @ A0).tocsr().astype(np.float32)
    A.sort_indices()
    b = (s * rng.uniform(-1, 1, A.shape[0])).astype(np.float32)
    return A, b, (1.0 / A.diagonal()).astype(np.float32)


def _gpu_jacobi(A, b, inv, index_dtype=np.int32, slice_mode=None, plan=True, x0=None, **kw):
    d, i, p = (torch.from_numpy(np.ascontiguousarray(a)).to(DEV) for a in _args(A, index_dtype))
    pl = _capi.Plan(p, A.shape[0], d.numel(), data=d, indices=i, n_cols=A.shape[1],
                    slice_mode=slice_mode) if plan else None
    out = _capi.gmres(d, i, p, torch.from_numpy(b).to(DEV),
                      None if x0 is None else torch.from_numpy(x0).to(DEV), plan=pl,
                      inv_diag=torch.from_numpy(inv).to(DEV), **kw)
    torch.cuda.synchronize()
    return (out[0].cpu().numpy(),) + tuple(out[1:])


def _jacobi_checks(A, b, inv, x, res, rtol, wx):
    dense = A.toarray().astype(np.float64)
    exact = np.linalg.solve(dense, b.astype(np.float64))
    cond = np.linalg.cond(np.diag(inv.astype(np.float64)) @ dense)
    assert np.linalg.norm(x - exact) <= 4 * cond * rtol * np.linalg.norm(exact)
    true_res = np.linalg.norm(b.astype(np.float64) - dense @ x.astype(np.float64))
    assert res <= rtol * np.linalg.norm(b) * (1 + 1e-5), res
    assert abs(true_res - res) <= 1e-5 * np.linalg.norm(b) + 1e-3 * res
    assert np.linalg.norm(x - wx) <= 1e-4 * np.linalg.norm(wx) + 4 * cond * rtol * \
        np.linalg.norm(exact)


@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
@pytest.mark.parametrize("restart", [1, 5, 20])
def test_gmres_jacobi_matches_oracle(index_dtype, restart):
    """Status equal to the oracle's, iterations within one cycle, x solving
    the system as well as the oracle's, on row-scaled random systems (and
    one with a starting guess)."""
    A, b, inv = _row_scaled(_random_nonsym(1200, seed=restart, density=0.005, shift=0.5),
                            seed=restart + 1)
    x0 = np.random.default_rng(restart).uniform(-0.1, 0.1, 1200).astype(np.float32)
    for guess in (None, x0):
        print(f"gmres jacobi random n=1200 restart={restart} x0={guess is not None} "
              f"{np.dtype(index_dtype).name}", flush=True)
        x, info, res, its = _gpu_jacobi(A, b, inv, index_dtype, x0=guess, rtol=1e-5,
                                        restart=restart, maxiter=20000)
        wx, winfo, wres, wits = orc.csr_gmres_jacobi(*_args(A, index_dtype), b, inv, guess,
                                                     rtol=1e-5, restart=restart, maxiter=20000)
        assert info == winfo == 0 and abs(its - wits) <= restart, (its, wits)
        _jacobi_checks(A, b, inv, x, res, 1e-5, wx)


@pytest.mark.parametrize("mode", ["blocks", "panels", "none"])
def test_gmres_jacobi_routes_and_reproducible(mode):
    A, b, inv = _row_scaled(convection_3d(40), seed=3)
    kw = {"plan": mode != "none",
          "slice_mode": {"blocks": _capi.SLICE_OFF, "panels": _capi.SLICE_PANELS,
                         "none": None}[mode]}
    print(f"gmres jacobi route={mode} n={A.shape[0]}", flush=True)
    r1 = _gpu_jacobi(A, b, inv, rtol=1e-5, restart=10, **kw)
    r2 = _gpu_jacobi(A, b, inv, rtol=1e-5, restart=10, **kw)
    assert r1[1:] == r2[1:] and r1[0].tobytes() == r2[0].tobytes()
    wx, winfo, wres, wits = orc.csr_gmres_jacobi(*_args(A), b, inv, rtol=1e-5, restart=10)
    assert r1[1] == winfo == 0 and abs(r1[3] - wits) <= 10 + wits // 20, (r1[3], wits)
    true_res = np.linalg.norm(b - A.astype(np.float64) @ r1[0].astype(np.float64))
    assert r1[2] <= 1e-5 * np.linalg.norm(b) * (1 + 1e-5)
    assert abs(true_res - r1[2]) <= 1e-5 * np.linalg.norm(b) + 1e-3 * r1[2]
    assert np.linalg.norm(r1[0].astype(np.float64) - wx) <= 1e-2 * np.linalg.norm(wx)


def test_gmres_jacobi_status_cases_match_oracle():
    """The Jacobi status rules against the oracle: a non-finite inverse
    diagonal entry or b (-3, residual +inf, no iterations), ||M r|| at most
    FLT_EPSILON (-1), a zero right-hand side, an exact x0, maxiter 0 and a
    short budget."""
    dense = np.diag([2.0, 3.0, 4.0, 5.0, 6.0, 7.0]).astype(np.float32)
    dense[0, 5] = 0.5
    dense[3, 1] = -0.25
    A = sp.csr_matrix(dense)
    A.sort_indices()
    inv = (1.0 / np.diag(dense)).astype(np.float32)
    b = np.linspace(-1.0, 1.5, 6, dtype=np.float32)
    bad_b = b.copy()
    bad_b[2] = np.nan
    bad_inv = inv.copy()
    bad_inv[1] = np.inf
    exact = np.linalg.solve(dense.astype(np.float64), b).astype(np.float32)
    bx = (dense.astype(np.float64) @ exact).astype(np.float32)
    cases = [(np.zeros(6, np.float32), inv, None, {}), (b, inv, None, {"maxiter": 0}),
             (b, inv, None, {"maxiter": 3, "restart": 2, "rtol": 1e-9}),
             (bad_b, inv, None, {}), (b, bad_inv, None, {}),
             (b, np.zeros(6, np.float32), None, {}), (b, np.full(6, 1e-30, np.float32), None, {}),
             (bx, inv, exact, {"atol": 1e-5}),
             (b, inv, None, {"rtol": 1e-6, "atol": 1e-7, "restart": 4, "maxiter": 32})]
    for rhs, iv, x0, kw in cases:
        print(f"gmres jacobi status case {kw} inv0={iv[0]} inv1={iv[1]}", flush=True)
        x, info, res, its = _gpu_jacobi(A, rhs, iv, x0=x0, **kw)
        wx, winfo, wres, wits = orc.csr_gmres_jacobi(*_args(A), rhs, iv, x0, **kw)
        assert (info, its) == (winfo, wits), (kw, info, its, winfo, wits)
        assert np.isinf(res) == np.isinf(wres) and np.isnan(res) == np.isnan(wres)
        if np.isfinite(wres):
            assert res == pytest.approx(wres, rel=1e-5, abs=1e-7)
        finite = np.isfinite(wx)
        np.testing.assert_array_equal(np.isfinite(x), finite)
        np.testing.assert_allclose(x[finite], wx[finite], rtol=1e-4, atol=1e-5)


def test_gmres_jacobi_api_on_gpu(gpu):
    """linalg.gmres with M = preconditioners.jacobi(A) on the device: the
    reference's left-preconditioned system and bounds
    (tests/test_linalg_preconditioners.py:1547-1597, 1600-1639)."""
    ms = gpu
    from mlx_sparse import linalg
    from mlx_sparse.linalg import preconditioners

    dense = np.array([[7.0, -2.0, 0.5, 0.0], [1.0, 5.5, -1.0, 0.25], [0.0, -0.5, 4.5, 1.0],
                      [0.25, 0.0, -0.75, 3.75]], np.float32)
    d, ix, ip = _csr(dense)
    csr = ms.csr_array((torch.from_numpy(d), torch.from_numpy(ix), torch.from_numpy(ip)),
                       shape=dense.shape, canonical=True)
    b = np.array([1.0, -2.0, 0.5, 3.0], np.float32)
    x, info = linalg.gmres(csr, b, M=preconditioners.jacobi(csr), rtol=1e-6, atol=1e-7,
                           restart=4, maxiter=32, return_info=True)
    assert info.status == 0 and info.preconditioner == "jacobi" and x.device.type == "cuda"
    xn = x.cpu().numpy().astype(np.float64)
    assert np.linalg.norm(dense @ xn - b) / np.linalg.norm(b) <= 2e-6
    np.testing.assert_allclose(xn, np.linalg.solve(dense.astype(np.float64), b), rtol=2e-4,
                               atol=2e-4)
