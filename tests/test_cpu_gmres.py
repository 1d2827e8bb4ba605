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
from test_oracle_gmres import _csr, _random_nonsym


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
    with pytest.raises(TypeError, match="identity"):
        ms.linalg.gmres(A, b, M=ms.linalg.preconditioners.jacobi(A))
    x, info = ms.linalg.gmres(A, b, M=ms.linalg.preconditioners.identity(A), maxiter=8)
    assert info == 0
    with pytest.raises(ValueError, match="length"):
        ms.linalg.gmres(A, torch.ones(3))
