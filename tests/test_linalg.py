"""``mlx_sparse.linalg.cg`` through the drop-in API, on the CPU (bit-exact
against the oracle) and the GPU (marked gpu; the device loop's own bar is in
test_gpu_solvers.py).  Ports the reference's docstring example and argument
checks (mlx_sparse/linalg/_iterative.py:69-200,
mlx_sparse/linalg/utils/iterative.py:49-70)."""

from __future__ import annotations

import numpy as np
import pytest
import scipy.sparse as sp
import torch

import mlx_sparse as ms
from mlx_sparse import linalg
from test_oracle_solvers import _args, laplacian_2d, random_spd

DEVICES = ["cpu", pytest.param("cuda", marks=pytest.mark.gpu)]


@pytest.fixture(params=DEVICES)
def dev(request, ms):
    prev = ms.default_torch_device()
    ms.use_cpu() if request.param == "cpu" else ms.use_gpu()
    yield request.param
    ms.use_gpu(prev.index or 0) if prev.type == "cuda" else ms.use_cpu()


def _csr(A):
    return ms.csr_array((A.data.astype(np.float32), A.indices.astype(np.int32),
                         A.indptr.astype(np.int32)), shape=A.shape, canonical=True)


def test_docstring_example(dev):
    # reference mlx_sparse/linalg/_iterative.py:150-167
    n = 16
    L = sp.diags([-1, 4, -1], [-1, 0, 1], shape=(n, n), format="csr").astype(np.float32)
    A = _csr(L)
    x, info = linalg.cg(A, torch.ones(n), rtol=1e-6)
    assert info == 0 and isinstance(info, int)
    np.testing.assert_allclose(L @ x.cpu().numpy(), np.ones(n), atol=1e-5)


def test_cg_api_equals_oracle_on_cpu(ms, oracle):
    ms.use_cpu()
    A = random_spd(400, 17)
    b = np.random.default_rng(3).standard_normal(400).astype(np.float32)
    x, info = linalg.cg(_csr(A), torch.from_numpy(b), rtol=1e-6, maxiter=500)
    wx, winfo, _, _ = oracle.csr_cg(*_args(A), b, rtol=1e-6, maxiter=500)
    assert info == winfo and x.numpy().tobytes() == wx.tobytes()
    inv = (1.0 / A.diagonal()).astype(np.float32)
    bb = 1e3 * b
    x, info = linalg.cg(_csr(A), torch.from_numpy(bb), rtol=1e-5,
                        M=linalg.preconditioners.jacobi(_csr(A)))
    wx, winfo, _, _ = oracle.csr_pcg_jacobi(*_args(A), bb, inv, rtol=1e-5)
    assert info == winfo == 0 and x.numpy().tobytes() == wx.tobytes()


def test_return_info_callback_and_budget(dev):
    A = _csr(laplacian_2d(12))
    b = torch.ones(144)
    seen = []
    x, info = linalg.cg(A, b, rtol=1e-6, return_info=True, callback=seen.append)
    assert isinstance(info, linalg.SolverInfo) and info.converged and int(info) == 0
    assert info.convergence_reason == "converged" and info.iterations > 0
    assert len(seen) == 1 and seen[0] is x
    x, info = linalg.cg(A, b, rtol=1e-9, maxiter=2, return_info=True)
    assert (info.status, info.iterations, info.convergence_reason) == (2, 2, "iteration_limit")
    x, info = linalg.cg(A, torch.zeros(144))
    assert info == 0 and not x.any()
    x, info = linalg.cg(A, b, x0=torch.full((144,), 0.5), rtol=1e-6)
    assert info == 0


def test_preconditioners(dev):
    A = _csr(random_spd(300, 5))
    b = 1e3 * torch.ones(300)
    for M in (linalg.preconditioners.identity(A), linalg.preconditioners.jacobi(A),
              linalg.preconditioners.diagonal(linalg.preconditioners.csr_diagonal(A)),
              1.0 / linalg.preconditioners.csr_diagonal(A)):
        x, info = linalg.cg(A, b, rtol=1e-5, M=M)
        assert info == 0
    _, info = linalg.cg(A, b, M=linalg.preconditioners.diagonal(-torch.ones(300)))
    assert info == -2
    Z = _csr(sp.csr_matrix(np.diag([1.0, 0.0, 2.0]).astype(np.float32)))
    with pytest.raises(ValueError, match="zero or near-zero"):
        linalg.preconditioners.jacobi(Z)
    assert bool((linalg.preconditioners.jacobi(Z, zero_policy="unit").inverse_diagonal
                 == torch.tensor([1.0, 1.0, 0.5], device=dev)).all())


def test_errors(dev):
    A = _csr(laplacian_2d(4))
    with pytest.raises(TypeError, match="CSRArray"):
        linalg.cg(torch.eye(3), torch.ones(3))
    with pytest.raises(ValueError, match="rank-1"):
        linalg.cg(A, torch.ones(16, 1))
    with pytest.raises(ValueError, match="b has length 3, expected 16"):
        linalg.cg(A, torch.ones(3))
    with pytest.raises(ValueError, match="x0 must have shape"):
        linalg.cg(A, torch.ones(16), x0=torch.ones(4))
    with pytest.raises(ValueError, match="maxiter must be non-negative"):
        linalg.cg(A, torch.ones(16), maxiter=-1)
    with pytest.raises(ValueError, match="square"):
        linalg.cg(ms.csr_array((torch.ones(2), torch.tensor([0, 1], dtype=torch.int32),
                                torch.tensor([0, 1, 2], dtype=torch.int32)), shape=(2, 3)),
                  torch.ones(2))
    with pytest.raises(TypeError, match="preconditioners"):
        linalg.cg(A, torch.ones(16), M="ilu")


@pytest.mark.gpu
def test_gpu_cg_matches_cpu_api(ms):
    A = random_spd(2000, 23)
    b = np.random.default_rng(5).standard_normal(2000).astype(np.float32)
    ms.use_cpu()
    xc, ic = linalg.cg(_csr(A), torch.from_numpy(b), rtol=1e-6, return_info=True)
    ms.use_gpu()
    try:
        xg, ig = linalg.cg(_csr(A), torch.from_numpy(b), rtol=1e-6, return_info=True)
        xg2, _ = linalg.cg(_csr(A), torch.from_numpy(b), rtol=1e-6)
    finally:
        ms.use_cpu()
    assert ic.status == ig.status == 0 and abs(ic.iterations - ig.iterations) <= 1
    assert xg.device.type == "cuda" and torch.equal(xg, xg2)
    np.testing.assert_allclose(xg.cpu().numpy(), xc.numpy(), rtol=0,
                               atol=1e-4 * float(xc.abs().max()))
