"""Derivatives of the CSR products and the transpose API, on the CPU and
(marked gpu) the HIP path.

Ports the reference's gradient tests (tests/test_grad.py:28-355: SpMV/SpMM
gradients in the dense operand and the stored values, complex64 rules,
float16/bfloat16 VJPs, batched helpers), its vmap tests
(tests/test_vmap_sparse_dense.py:137-279) and transpose tests
(tests/test_transpose.py:23-65).  Expected values come from torch's dense
products under autograd in float64/complex128, an independent formulation
of the same derivatives, with the reference tests' tolerances (1e-5; 5e-3
float16, 3e-2 bfloat16); known answers are checked exactly.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import mlx_sparse as ms
from mlx_sparse import runtime

DEVICES = ["cpu", pytest.param("cuda", marks=pytest.mark.gpu)]

COL = np.array([0, 2, 1, 3], np.int32)
PTR = np.array([0, 2, 2, 4], np.int32)
DATA = np.array([2.0, -1.0, 4.0, 5.0], np.float32)


@pytest.fixture(params=DEVICES)
def dev(request, ms):
    prev = ms.default_torch_device()
    if request.param == "cpu":
        ms.use_cpu()
    else:
        ms.use_gpu()
    yield torch.device(request.param)
    if prev.type == "cuda":
        ms.use_gpu(prev.index or 0)
    else:
        ms.use_cpu()


def _t(a, dev, dtype=None):
    a = np.asarray(a)
    if a.dtype == np.float64:
        a = a.astype(np.float32)
    elif a.dtype == np.complex128:
        a = a.astype(np.complex64)
    return torch.as_tensor(a).to(dev, dtype=dtype)


def _csr(values, dev, indices=COL, indptr=PTR, shape=(3, 4)):
    return ms.csr_array((values, _t(indices, dev), _t(indptr, dev)), shape=shape,
                        sorted_indices=True, canonical=True)


def _dense(values, dev, indices=COL, indptr=PTR, shape=(3, 4)):
    rows = np.repeat(np.arange(shape[0]), np.diff(indptr))
    D = torch.zeros(shape, dtype=values.dtype, device=values.device)
    return D.index_put((_t(rows, dev), _t(indices, dev).long()), values, accumulate=True)


def _close(got, want, tol=1e-5):
    got = got.detach().cpu()
    want = want.detach().cpu().to(got.dtype)
    torch.testing.assert_close(got, want, rtol=tol, atol=tol)


def test_matvec_rhs_gradient_kat(dev):
    # reference tests/test_grad.py:28-50
    A = _csr(_t(DATA, dev), dev)
    x = _t([3.0, 10.0, 7.0, -2.0], dev).requires_grad_()
    (A @ x).pow(2).sum().backward()
    assert x.grad.cpu().tolist() == [-4.0, 240.0, 2.0, 300.0]


def test_matmul_rhs_gradient(dev):
    # reference tests/test_grad.py:53-85
    A = _csr(_t(DATA, dev), dev)
    X = _t(np.arange(8, dtype=np.float32).reshape(4, 2) / 3.0, dev).requires_grad_()
    (A @ X).pow(2).sum().backward()
    Xd = X.detach().double().requires_grad_()
    (_dense(_t(DATA, dev).double(), dev) @ Xd).pow(2).sum().backward()
    _close(X.grad, Xd.grad)


def test_matvec_data_and_rhs_gradients(dev):
    # reference tests/test_grad.py:180-223
    values = _t(DATA, dev).requires_grad_()
    x = _t([3.0, 10.0, 7.0, -2.0], dev).requires_grad_()
    (_csr(values, dev) @ x).pow(2).sum().backward()
    assert values.grad.cpu().tolist() == [-6.0, -14.0, 600.0, -120.0]
    assert x.grad.cpu().tolist() == [-4.0, 240.0, 2.0, 300.0]


def test_matmul_complex_data_and_rhs_gradients(dev):
    # reference tests/test_grad.py:226-278 (loss = sum |Y|^2)
    col = np.array([0, 2, 1, 3], np.int32)
    ptr = np.array([0, 2, 3, 4], np.int32)
    data = np.array([1.0 + 0.5j, -2.0 + 1.0j, 0.25 - 1.5j, 3.0 + 0.25j], np.complex64)
    rhs = np.array([[1.0 - 0.5j, 2.0 + 0.25j], [-1.0 + 1.5j, 0.5 - 0.75j],
                    [2.0 + 0.0j, -3.0 + 0.5j], [0.25 - 2.0j, 1.0 + 1.0j]], np.complex64)
    values = _t(data, dev).requires_grad_()
    R = _t(rhs, dev).requires_grad_()
    Y = _csr(values, dev, col, ptr) @ R
    (Y * Y.conj()).real.sum().backward()
    vd = _t(data, dev).to(torch.complex128).requires_grad_()
    Rd = _t(rhs, dev).to(torch.complex128).requires_grad_()
    Yd = _dense(vd, dev, col, ptr) @ Rd
    (Yd * Yd.conj()).real.sum().backward()
    _close(values.grad, vd.grad)
    _close(R.grad, Rd.grad)


def test_matvec_complex_jvp_and_vjp(dev):
    # reference tests/test_grad.py:281-316
    data = _t(np.array([1.0 + 0.5j, -2.0 + 1.0j, 3.0 - 0.25j], np.complex64), dev)
    col = np.array([0, 2, 1], np.int32)
    ptr = np.array([0, 2, 3], np.int32)
    A = _csr(data, dev, col, ptr, (2, 3))
    D = _dense(data.to(torch.complex128), dev, col, ptr, (2, 3))
    x = _t(np.array([1.0 - 1.0j, 2.0 + 0.5j, -1.0j], np.complex64), dev)
    tangent = _t(np.array([0.25 + 0.5j, -1.0 + 0.75j, 2.0 - 0.5j], np.complex64), dev)
    cot = _t(np.array([2.0 - 1.0j, -0.5 + 3.0j], np.complex64), dev)
    _, jv = torch.func.jvp(lambda v: A @ v, (x,), (tangent,))
    _, jd = torch.func.jvp(lambda v: D @ v, (x.to(torch.complex128),),
                           (tangent.to(torch.complex128),))
    _close(jv, jd)
    _, vjp_fn = torch.func.vjp(lambda v: A @ v, x)
    _, vjp_d = torch.func.vjp(lambda v: D @ v, x.to(torch.complex128))
    _close(vjp_fn(cot)[0], vjp_d(cot.to(torch.complex128))[0])


@pytest.mark.parametrize(("dtype", "tol"), [(torch.float16, 5e-3), (torch.bfloat16, 3e-2)])
def test_matvec_low_precision_vjp(dev, dtype, tol):
    # reference tests/test_grad.py:319-355
    col = np.array([0, 3, 1, 3, 2, 4], np.int64)
    ptr = np.array([0, 2, 3, 5, 6], np.int64)
    data = _t(np.array([2.0, -1.0, 0.5, 3.0, -2.5, 1.25], np.float32), dev, dtype)
    x = _t(np.array([1.0, -0.5, 2.0, 0.75, -1.25], np.float32), dev, dtype)
    cot = _t(np.array([1.0, -0.5, 2.0, 0.75], np.float32), dev, dtype)
    A = _csr(data, dev, col, ptr, (4, 5))
    _, vjp_fn = torch.func.vjp(lambda v: A @ v, x)
    want = _dense(data.double(), dev, col, ptr, (4, 5)).T @ cot.double()
    _close(vjp_fn(cot)[0].float(), want.float(), tol)


def test_batched_matvec_gradients(dev):
    # reference tests/test_grad.py:88-131
    values = _t(DATA, dev).requires_grad_()
    rhs = _t(np.arange(24, dtype=np.float32).reshape(2, 3, 4) / 7.0, dev).requires_grad_()
    ms.csr_batched_matvec(_csr(values, dev), rhs).pow(2).sum().backward()
    vd = _t(DATA, dev).double().requires_grad_()
    rd = rhs.detach().double().requires_grad_()
    (rd @ _dense(vd, dev).T).pow(2).sum().backward()
    _close(values.grad, vd.grad)
    _close(rhs.grad, rd.grad)


def test_batched_matmul_gradients(dev):
    # reference tests/test_grad.py:134-177
    values = _t(DATA, dev).requires_grad_()
    rhs = _t(np.arange(24, dtype=np.float32).reshape(2, 4, 3) / 9.0, dev).requires_grad_()
    ms.csr_batched_matmul(_csr(values, dev), rhs).pow(2).sum().backward()
    vd = _t(DATA, dev).double().requires_grad_()
    rd = rhs.detach().double().requires_grad_()
    (_dense(vd, dev)[None] @ rd).pow(2).sum().backward()
    _close(values.grad, vd.grad)
    _close(rhs.grad, rd.grad)


def test_batched_products_equal_batched_kernels_when_tracked(dev):
    # the tracked batched route must give the batched kernels' values bit for bit
    rng = np.random.default_rng(3)
    n, m = 50, 40
    lengths = rng.integers(0, 9, n)
    ptr = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    col = rng.integers(0, m, ptr[-1]).astype(np.int32)
    values = _t(rng.standard_normal(ptr[-1]).astype(np.float32), dev)
    A = _csr(values, dev, col, ptr, (n, m))
    V = _t(rng.standard_normal((5, m)).astype(np.float32), dev)
    M = _t(rng.standard_normal((3, m, 4)).astype(np.float32), dev)
    plain_v, plain_m = ms.csr_batched_matvec(A, V), ms.csr_batched_matmul(A, M)
    Vg, Mg = V.clone().requires_grad_(), M.clone().requires_grad_()
    assert torch.equal(ms.csr_batched_matvec(A, Vg).detach(), plain_v)
    assert torch.equal(ms.csr_batched_matmul(A, Mg).detach(), plain_m)


def test_func_grad_and_vmap(dev):
    A = _csr(_t(DATA, dev), dev)
    D = _dense(_t(DATA, dev).double(), dev)
    x = _t([3.0, 10.0, 7.0, -2.0], dev)
    g = torch.func.grad(lambda v: (A @ v).pow(2).sum())(x)
    assert g.cpu().tolist() == [-4.0, 240.0, 2.0, 300.0]
    # reference tests/test_vmap_sparse_dense.py:137-195
    X = _t(np.arange(20, dtype=np.float32).reshape(5, 4) / 3.0, dev)
    _close(torch.func.vmap(lambda v: A @ v)(X), X.double() @ D.T)
    _close(torch.func.vmap(lambda v: A @ v, in_dims=1, out_dims=1)(X.T.contiguous()),
           (X.double() @ D.T).T)
    M = _t(np.arange(40, dtype=np.float32).reshape(5, 4, 2) / 5.0, dev)
    _close(torch.func.vmap(lambda r: A @ r)(M), D @ M.double())
    # nested: vmap over the explicit batched helper
    B = _t(np.arange(60, dtype=np.float32).reshape(3, 5, 4) / 7.0, dev)
    _close(torch.func.vmap(lambda b: ms.csr_batched_matvec(A, b))(B), B.double() @ D.T)


def test_vmap_rejects_mapped_sparse_values(dev):
    # reference tests/test_vmap_sparse_dense.py:244-267
    V = _t(np.stack([DATA, 2 * DATA]), dev)
    x = _t([1.0, 2.0, 3.0, 4.0], dev)
    with pytest.raises(ValueError, match="batching only the dense RHS"):
        torch.func.vmap(lambda v: _csr(v, dev) @ x)(V)


def test_vmap_zero_nnz_shapes(dev):
    # reference tests/test_vmap_sparse_dense.py:227-241
    A = ms.csr_array((_t(np.zeros(0, np.float32), dev), _t(np.zeros(0, np.int32), dev),
                      _t(np.zeros(4, np.int32), dev)), shape=(3, 5))
    out = torch.func.vmap(lambda v: A @ v)(_t(np.ones((2, 5), np.float32), dev))
    assert out.shape == (2, 3) and not out.any()
    out = torch.func.vmap(lambda r: A @ r)(_t(np.ones((2, 5, 4), np.float32), dev))
    assert out.shape == (2, 3, 4) and not out.any()


def test_transpose_api(dev, oracle):
    # reference tests/test_transpose.py:23-65
    A = _csr(_t(DATA, dev), dev)
    T = A.T
    assert T.shape == (4, 3) and T.sorted_indices and T.has_canonical_format
    assert torch.equal(T.todense().cpu(), A.todense().cpu().T)
    assert T is A.T  # cached on the immutable array
    data = _t(np.array([1.0 + 2.0j, 3.0 - 4.0j, -2.0 + 1.0j], np.complex64), dev)
    C = _csr(data, dev, np.array([0, 2, 1], np.int32), np.array([0, 2, 3], np.int32), (2, 3))
    assert torch.equal(C.H.todense().cpu(), C.todense().cpu().conj().T)
    assert torch.equal(C.conj().data.cpu(), data.cpu().conj())
    assert torch.equal(C.conjugate().data.cpu(), data.cpu().conj())
    # A.T @ y is SpMV over the transpose: equal to the oracle's route
    y = _t([1.5, -2.0, 0.25], dev)
    got = (A.T @ y).cpu().numpy()
    td, ti, tp = oracle.csr_transpose(DATA, COL, PTR, 3, 4)
    np.testing.assert_array_equal(got, oracle.csr_matvec(td, ti, tp, y.cpu().numpy(), 4))
    # the transposed products without a transpose
    _close(ms.csr_matvec_transpose(A, y), A.todense().double().T @ y.double())
    Y = _t(np.arange(6, dtype=np.float32).reshape(3, 2), dev)
    _close(ms.csr_matmul_transpose(A, Y), A.todense().double().T @ Y.double())
    with pytest.raises(ValueError, match="expects x of shape"):
        ms.csr_matvec_transpose(A, _t([1.0, 2.0], dev))
    with pytest.raises(TypeError, match="same dtype"):
        ms.csr_matvec_transpose(A, y.double())


def test_transpose_of_transpose_is_identity(dev):
    rng = np.random.default_rng(5)
    n, m = 70, 45
    lengths = rng.integers(0, 7, n)
    ptr = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    col = np.concatenate([np.sort(rng.choice(m, size=int(k), replace=False)) for k in lengths]
                         ).astype(np.int64)
    A = _csr(_t(rng.standard_normal(ptr[-1]).astype(np.float32), dev), dev, col, ptr, (n, m))
    TT = A.T.T
    assert torch.equal(TT.indptr.cpu(), A.indptr.cpu())
    assert torch.equal(TT.indices.cpu(), A.indices.cpu())
    assert torch.equal(TT.data.cpu(), A.data.cpu())


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.complex64])
def test_gpu_adjoint_routes(ms, dtype):
    """The three GPU routes of A^H g agree; the transpose route equals
    ``A.H @ g`` bit for bit, and "auto" switches to the cached transpose on a
    matrix's second adjoint product."""
    ms.use_gpu()
    try:
        rng = np.random.default_rng(7)
        n, m = 3000, 2000
        lengths = rng.integers(0, 30, n)
        ptr = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
        col = rng.integers(0, m, ptr[-1]).astype(np.int32)
        v = rng.standard_normal(ptr[-1])
        if dtype == torch.complex64:
            v = v + 1j * rng.standard_normal(ptr[-1])
        data = torch.as_tensor(v).to("cuda", dtype)
        g = torch.as_tensor(rng.standard_normal(n)).to("cuda", dtype)
        x = torch.zeros(m, dtype=dtype, device="cuda")

        def grad_x(A):
            xr = x.clone().requires_grad_()
            (A @ xr).backward(g)
            return xr.grad

        out = {}
        for mode in ("atomic", "transpose", "auto"):
            A = _csr(data, "cuda", col, ptr, (n, m))
            with runtime.context(gpu_adjoint=mode):
                first = grad_x(A)
                second = grad_x(A)
            out[mode] = (first, second)
            key = ("H" if dtype == torch.complex64 else "T", "cuda:0")
            assert (key in A._cache) == (mode != "atomic")
        want = (_csr(data, "cuda", col, ptr, (n, m)).H @ g)
        assert torch.equal(out["transpose"][0], want) and torch.equal(out["transpose"][1], want)
        assert torch.equal(out["auto"][1], want)
        scale = (_csr(data.abs().to(dtype), "cuda", col, ptr, (n, m)).T @ g.abs().to(dtype)).abs()
        for got in (out["atomic"][0], out["atomic"][1], out["auto"][0]):
            assert torch.all((got - want).abs() <= 1e-5 * scale.real + 1e-30)
    finally:
        ms.use_cpu()
