"""HIP conjugate gradient solvers (msx_csr_cg, msx_csr_pcg_jacobi) against
the oracle through the C ABI.

The device loop follows the reference's arithmetic (float SpMV from zero,
double dot products and updates; float scalars for Jacobi PCG) but adds
its dot products per workgroup, so the rounding of the double sums differs
from the sequential loop.  The bar:

- status and iteration count equal the oracle's (iterations within one on
  the larger systems, where a double-rounding difference can move the
  crossing of the tolerance by a step);
- x solves the system as well as the oracle's x: error against a float64
  dense (or oracle) solution within the CG bound, true residual at the
  tolerance, reported residual equal to the true one to float32 rounding;
- the status cases (zero right-hand side, maxiter 0 and short budgets,
  non-finite input, indefinite matrix, non-positive preconditioner) give the
  oracle's status, iterations and residual exactly;
- a solve is reproducible: two runs give the same bits;
- every SpMV route (row blocks, XCD slices, LDS panels, no plan) runs
  inside the loop.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import _capi
from oracle import oracle as orc
from test_oracle_solvers import _args, laplacian_2d, random_spd

pytestmark = pytest.mark.gpu

DEV = "cuda"


def poisson_3d(g):
    import scipy.sparse as sp

    one = sp.diags([-1, 2, -1], [-1, 0, 1], shape=(g, g))
    eye = sp.identity(g)
    A = (sp.kron(sp.kron(one, eye), eye) + sp.kron(sp.kron(eye, one), eye)
         + sp.kron(sp.kron(eye, eye), one)).tocsr()
    A.sort_indices()
    return A.astype(np.float32)


def _dev(A, index_dtype=np.int32):
    return tuple(torch.from_numpy(a).to(DEV) for a in _args(A, index_dtype))


def _gpu(A, b, index_dtype=np.int32, slice_mode=None, plan=True, **kw):
    d, i, p = _dev(A, index_dtype)
    pl = _capi.Plan(p, A.shape[0], d.numel(), data=d, indices=i, n_cols=A.shape[1],
                    slice_mode=slice_mode) if plan else None
    inv = kw.pop("inv_diag", None)
    x0 = kw.pop("x0", None)
    out = _capi.cg(d, i, p, torch.from_numpy(b).to(DEV),
                   None if x0 is None else torch.from_numpy(x0).to(DEV), plan=pl,
                   inv_diag=None if inv is None else torch.from_numpy(inv).to(DEV), **kw)
    torch.cuda.synchronize()
    return (out[0].cpu().numpy(),) + tuple(out[1:]) + ((pl.info().n_panels, pl.info().n_slices)
                                                        if pl else (0, 0),)


@pytest.mark.parametrize("name", ["laplacian", "random"])
@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_cg_matches_oracle_small(name, index_dtype):
    A = laplacian_2d(32) if name == "laplacian" else random_spd(900, 13)
    n = A.shape[0]
    b = np.random.default_rng(8).standard_normal(n).astype(np.float32)
    rtol = 1e-6
    print(f"cg {name} {np.dtype(index_dtype).name} n={n}", flush=True)
    x, info, res, its, _ = _gpu(A, b, index_dtype, rtol=rtol)
    wx, winfo, wres, wits = orc.csr_cg(*_args(A, index_dtype), b, rtol=rtol)
    assert info == winfo == 0 and abs(its - wits) <= 1
    A64 = A.astype(np.float64)
    exact = np.linalg.solve(A64.toarray(), b.astype(np.float64))
    cond = np.linalg.cond(A64.toarray())
    assert np.linalg.norm(x - exact) <= 4 * cond * rtol * np.linalg.norm(exact)
    true_res = np.linalg.norm(b.astype(np.float64) - A64 @ x.astype(np.float64))
    assert abs(true_res - res) <= 1e-5 * np.linalg.norm(b) + 1e-3 * res
    assert res <= rtol * np.linalg.norm(b) * (1 + 1e-6)


@pytest.mark.parametrize("mode", ["blocks", "slices", "panels", "none"])
def test_cg_every_spmv_route_and_reproducible(mode):
    A = poisson_3d(40)
    n = A.shape[0]
    b = np.random.default_rng(9).standard_normal(n).astype(np.float32)
    kw = {"plan": mode != "none",
          "slice_mode": {"blocks": _capi.SLICE_OFF, "slices": _capi.SLICE_ON,
                         "panels": _capi.SLICE_PANELS, "none": None}[mode]}
    print(f"cg poisson 40^3 route={mode}", flush=True)
    x1, info1, res1, its1, kinds = _gpu(A, b, rtol=1e-6, **kw)
    x2, info2, res2, its2, _ = _gpu(A, b, rtol=1e-6, **kw)
    if mode == "panels":
        assert kinds[0] > 0
    if mode == "slices":
        assert kinds[1] > 0
    assert (info1, its1) == (info2, its2) and res1 == res2 and x1.tobytes() == x2.tobytes()
    wx, winfo, wres, wits = orc.csr_cg(*_args(A), b, rtol=1e-6)
    assert info1 == winfo == 0 and abs(its1 - wits) <= 1
    ref = np.linalg.norm(wx.astype(np.float64))
    assert np.linalg.norm(x1.astype(np.float64) - wx) <= 1e-4 * ref


def test_pcg_jacobi_matches_oracle():
    A = random_spd(1200, 21)
    n = A.shape[0]
    b = (1e3 * np.random.default_rng(10).standard_normal(n)).astype(np.float32)
    inv = (1.0 / A.diagonal()).astype(np.float32)
    print("pcg jacobi n=1200", flush=True)
    x, info, res, its, _ = _gpu(A, b, inv_diag=inv, rtol=1e-5)
    wx, winfo, wres, wits = orc.csr_pcg_jacobi(*_args(A), b, inv, rtol=1e-5)
    assert info == winfo == 0 and abs(its - wits) <= 1
    np.testing.assert_allclose(x, wx, rtol=0, atol=1e-4 * np.abs(wx).max())
    # the reference's -1 rule on a tiny right-hand side, decided at step one
    L = laplacian_2d(6)
    m = L.shape[0]
    got = _gpu(L, np.full(m, 1e-5, np.float32), inv_diag=np.full(m, 0.25, np.float32),
               rtol=1e-6)
    want = orc.csr_pcg_jacobi(*_args(L), np.full(m, 1e-5, np.float32),
                              np.full(m, 0.25, np.float32), rtol=1e-6)
    assert got[1:4] == want[1:]


def test_status_cases_equal_oracle():
    A = laplacian_2d(8)
    n = A.shape[0]
    x0 = (np.arange(n, dtype=np.float32) % 3)
    bad = np.ones(n, np.float32)
    bad[5] = np.nan
    cases = [
        (A, np.zeros(n, np.float32), {}),
        (A, (A @ x0).astype(np.float32), {"x0": x0}),
        (A, np.ones(n, np.float32), {"maxiter": 0}),
        (A, np.ones(n, np.float32), {"maxiter": 3, "rtol": 1e-8}),
        (A, bad, {}),
    ]
    for M, b, kw in cases:
        print(f"status case {sorted(kw)}", flush=True)
        got = _gpu(M, b, **dict(kw))
        want = orc.csr_cg(*_args(M), b, **kw)
        assert (got[1], got[3]) == (want[1], want[3]), kw
        if want[1] in (0, 1) and want[3] == 0:
            assert got[2] == want[2] and got[0].tobytes() == want[0].tobytes()
    import scipy.sparse as sp

    D = sp.diags(np.array([1.0, -1.0], np.float32)).tocsr()
    got = _gpu(D, np.ones(2, np.float32), plan=False)
    assert (got[1], got[3]) == (-1, 0)
    got = _gpu(A, np.ones(n, np.float32), inv_diag=np.full(n, -0.25, np.float32))
    assert (got[1], got[3]) == (-2, 0)
    got = _gpu(A, bad, inv_diag=np.full(n, 0.25, np.float32))
    assert got[1] == -3


def test_cg_poisson_64_cubed():
    A = poisson_3d(64)
    n = A.shape[0]
    b = np.ones(n, np.float32)
    print(f"cg poisson 64^3 n={n}", flush=True)
    x, info, res, its, _ = _gpu(A, b, rtol=1e-6)
    wx, winfo, wres, wits = orc.csr_cg(*_args(A), b, rtol=1e-6)
    assert info == winfo == 0 and abs(its - wits) <= 1
    # the true residual of a float32 x bottoms out at the rounding of x
    # (|A||x| * 2^-24 per row, ~0.08 here), for the oracle's x as well
    A64 = A.astype(np.float64)
    true_res = np.linalg.norm(b - A64 @ x.astype(np.float64))
    oracle_res = np.linalg.norm(b - A64 @ wx.astype(np.float64))
    assert true_res <= 1.5 * oracle_res + 1e-6 * np.linalg.norm(b)
    assert np.linalg.norm(x.astype(np.float64) - wx) <= 1e-4 * np.linalg.norm(wx)


def test_solver_errors():
    d = torch.ones(1, device=DEV)
    i = torch.zeros(1, dtype=torch.int32, device=DEV)
    p = torch.tensor([0, 1], dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError, match="maxiter must be non-negative"):
        _capi.cg(d, i, p, torch.ones(1, device=DEV), maxiter=-1)
    other = _capi.Plan(torch.tensor([0, 1, 2], dtype=torch.int32, device=DEV), 2, 2)
    with pytest.raises(RuntimeError, match="different matrix"):
        _capi.cg(d, i, p, torch.ones(1, device=DEV), plan=other)
