"""Native CPU solvers (msx_csr_cg_cpu, msx_csr_pcg_jacobi_cpu) against the
oracle through the C ABI: the same sequential loops, so x, info, residual and
iteration count agree bit for bit."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import _capi
from test_oracle_solvers import _args, laplacian_2d, random_spd


def _native(A, b, index_dtype=np.int32, **kw):
    d, i, p = (torch.from_numpy(a) for a in _args(A, index_dtype))
    inv = kw.pop("inv_diag", None)
    x0 = kw.pop("x0", None)
    return _capi.cg(d, i, p, torch.from_numpy(b), None if x0 is None else torch.from_numpy(x0),
                    inv_diag=None if inv is None else torch.from_numpy(inv), **kw)


@pytest.mark.parametrize("name", ["laplacian", "random"])
@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_cg_cpu_equals_oracle(oracle, name, index_dtype):
    A = laplacian_2d(20) if name == "laplacian" else random_spd(700, 11)
    b = np.random.default_rng(4).standard_normal(A.shape[0]).astype(np.float32)
    for kw in ({"rtol": 1e-6}, {"rtol": 1e-3, "atol": 0.5}, {"maxiter": 7, "rtol": 1e-9}):
        x, info, res, its = _native(A, b, index_dtype, **kw)
        wx, winfo, wres, wits = oracle.csr_cg(*_args(A, index_dtype), b, **kw)
        assert (info, its) == (winfo, wits)
        assert np.float32(res).tobytes() == np.float32(wres).tobytes()
        assert x.numpy().tobytes() == wx.tobytes()


def test_pcg_jacobi_cpu_equals_oracle(oracle):
    A = random_spd(600, 5)
    b = (1e3 * np.random.default_rng(6).standard_normal(A.shape[0])).astype(np.float32)
    inv = (1.0 / A.diagonal()).astype(np.float32)
    x0 = np.full(A.shape[0], 0.5, np.float32)
    for kw in ({"rtol": 1e-5}, {"rtol": 1e-8, "maxiter": 5}):
        x, info, res, its = _native(A, b, inv_diag=inv, x0=x0, **kw)
        wx, winfo, wres, wits = oracle.csr_pcg_jacobi(*_args(A), b, inv, x0=x0, **kw)
        assert (info, its) == (winfo, wits)
        assert np.float32(res).tobytes() == np.float32(wres).tobytes()
        assert x.numpy().tobytes() == wx.tobytes()


def test_cpu_status_cases_equal_oracle(oracle):
    A = laplacian_2d(6)
    n = A.shape[0]
    cases = [(np.zeros(n, np.float32), {}), (np.ones(n, np.float32), {"maxiter": 0})]
    bad = np.ones(n, np.float32)
    bad[3] = np.inf
    cases.append((bad, {}))
    for b, kw in cases:
        got = _native(A, b, **kw)[1:]
        want = oracle.csr_cg(*_args(A), b, **kw)[1:]
        assert got[0] == want[0] and got[2] == want[2]
    got = _native(A, np.ones(n, np.float32), inv_diag=np.full(n, -1.0, np.float32))
    assert got[1] == -2


def test_cpu_solver_errors():
    d = torch.ones(1)
    i = torch.zeros(1, dtype=torch.int32)
    p = torch.tensor([0, 1], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="maxiter must be non-negative"):
        _capi.cg(d, i, p, torch.ones(1), maxiter=-1)
    res = _capi.SolverResult()
    st = _capi.lib().msx_csr_cg_cpu(0, 0, 0, None, None, p.data_ptr(), None, None, None, 1e-5,
                                    0.0, 1, None)
    assert st == _capi.EINVAL and "non-empty square" in _capi.last_error()
    assert res.info == 0
