"""The drop-in API on the CPU device (``ms.use_cpu()``): the reference's path
tests ported to torch tensors, and the native CPU kernels compared with the
oracle bit for bit (same stored-order sums, same accumulator rules)."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from _util import storage, to_numpy, widen

GOLDEN = Path(__file__).resolve().parent / "golden"


def _kat(ms, data=(2.0, -1.0, 4.0, 5.0), dtype=np.float32):
    return ms.csr_array((np.array(data, dtype=dtype), np.array([0, 2, 1, 3], np.int32),
                         np.array([0, 2, 2, 4], np.int32)), shape=(3, 4))


def test_matvec_hand_computed(cpu):
    # reference tests/test_csr_matvec.py:25-36
    y = _kat(cpu) @ np.array([3.0, 10.0, 7.0, -2.0], np.float32)
    assert y.device.type == "cpu"
    np.testing.assert_array_equal(y.numpy(), [-1.0, 0.0, 30.0])


def test_matmul_hand_computed(cpu):
    # reference tests/test_csr_matmul.py:25-45
    out = _kat(cpu) @ np.array([[3, 1], [10, -2], [7, 4], [-2, 6]], np.float32)
    np.testing.assert_array_equal(out.numpy(), [[-1, -2], [0, 0], [30, 22]])


def test_noncontiguous_inputs(cpu):
    # reference tests/test_csr_matvec.py:318-333
    data = torch.tensor([99.0, 2.0, 99.0, -1.0, 99.0, 4.0, 99.0, 5.0])[1::2]
    idx = torch.tensor([9, 0, 9, 2, 9, 1, 9, 3], dtype=torch.int32)[1::2]
    x = torch.tensor([99.0, 3.0, 99.0, 10.0, 99.0, 7.0, 99.0, -2.0])[1::2]
    A = cpu.csr_array((data, idx, torch.tensor([0, 2, 2, 4], dtype=torch.int32)), shape=(3, 4))
    np.testing.assert_array_equal((A @ x).numpy(), [-1.0, 0.0, 30.0])


def test_errors(cpu):
    # reference tests/test_csr_matvec.py:336-361, test_dtypes.py:113-124,
    # test_csr_matmul.py:520-535
    A = cpu.csr_array((np.ones(1, np.float32), np.zeros(1, np.int32), np.array([0, 1], np.int32)),
                      shape=(1, 2))
    with pytest.raises(ValueError, match="n_cols"):
        A @ torch.ones(1)
    with pytest.raises(TypeError, match="dtype must be one"):
        A @ torch.ones(2, dtype=torch.int32)
    with pytest.raises(TypeError, match="same dtype"):
        A @ torch.ones(2, dtype=torch.float16)
    with pytest.raises(ValueError, match="n_cols"):
        A @ torch.ones((1, 2))
    with pytest.raises(TypeError, match="indices and indptr must have the same dtype"):
        cpu.csr_array((np.ones(1, np.float32), np.zeros(1, np.int64), np.array([0, 1], np.int32)),
                      shape=(1, 2))
    with pytest.raises(ValueError, match="indptr must have shape"):
        cpu.csr_array((np.ones(1, np.float32), np.zeros(1, np.int32), np.array([0, 1, 1], np.int32)),
                      shape=(1, 2))
    with pytest.raises(ValueError, match="indices must be in bounds"):
        cpu.csr_array((np.ones(1, np.float32), np.array([5], np.int32), np.array([0, 1], np.int32)),
                      shape=(1, 2), validate="full")


def test_cpp_layer_error_texts(cpu):
    # C++ op layer texts (reference src/common/common.cpp:104-177)
    from mlx_sparse._ext_loader import extension

    ext = extension()
    d = torch.ones(2)
    i = torch.zeros(2, dtype=torch.int32)
    p = torch.tensor([0, 2], dtype=torch.int32)
    with pytest.raises(ValueError, match="csr_matvec x must have size 3, got 2."):
        ext.csr_matvec(d, i, p, torch.ones(2), 1, 3)
    with pytest.raises(ValueError, match="csr_matvec data and csr_matvec x must have the same dtype"):
        ext.csr_matvec(d, i, p, torch.ones(3, dtype=torch.float16), 1, 3)
    with pytest.raises(ValueError, match="csr_matvec indptr must have size 3, got 2."):
        ext.csr_matvec(d, i, p, torch.ones(3), 2, 3)
    with pytest.raises(ValueError, match="must be rank-1, got rank 2"):
        ext.csr_matvec(d, i, p, torch.ones((3, 1)), 1, 3)
    with pytest.raises(ValueError, match="shape dimensions must be non-negative"):
        ext.csr_matvec(d, i, p, torch.ones(3), -1, 3)
    with pytest.raises(ValueError, match="rhs first dimension must equal"):
        ext.csr_matmul(d, i, p, torch.ones((2, 2)), 1, 3)


@pytest.mark.parametrize("dtype,tol", [("float16", 5e-3), ("float32", 1e-5), ("complex64", 1e-5)])
def test_dtype_kats(cpu, dtype, tol):
    # reference tests/test_dtypes.py:24-61
    vals = np.array([2.0, -1.0, 4.0, 5.0])
    x = np.array([3.0, 10.0, 7.0, -2.0])
    if dtype == "complex64":
        vals = vals + np.array([1j, -2j, 0.5j, 3j])
        x = x + np.array([-1j, 2j, 0j, -0.5j])
    v, xs = storage(vals, dtype), storage(x, dtype)
    A = cpu.csr_array((v, np.array([0, 2, 1, 3], np.int32), np.array([0, 2, 2, 4], np.int32)),
                      shape=(3, 4))
    want = np.array([v[0] * xs[0] + v[1] * xs[2], 0, v[2] * xs[1] + v[3] * xs[3]])
    np.testing.assert_allclose((A @ torch.from_numpy(xs)).numpy(), want, rtol=tol, atol=tol)


def test_bfloat16_returns_bfloat16(cpu):
    # reference tests/test_dtypes.py:64-77
    A = cpu.csr_array((torch.tensor([2.0, -1.0], dtype=torch.bfloat16),
                       torch.tensor([0, 1], dtype=torch.int32), torch.tensor([0, 2], dtype=torch.int32)),
                      shape=(1, 2))
    y = A @ torch.tensor([3.0, 7.0], dtype=torch.bfloat16)
    assert y.dtype == torch.bfloat16 and y.float().item() == -1.0


@pytest.mark.parametrize("k", [1, 2, 4, 8, 16, 32])
def test_widths_serial_parallel(cpu, oracle, k):
    # reference tests/test_csr_matmul.py:128-154 (serial == parallel, bitwise)
    z = np.load(GOLDEN / "scipy_cases.npz")
    pre = f"widths{k}"
    shape = tuple(int(v) for v in z[f"{pre}.shape"])
    A = cpu.csr_array((z[f"{pre}.data"], z[f"{pre}.indices"], z[f"{pre}.indptr"]), shape=shape)
    X = torch.from_numpy(z[f"{pre}.X"])
    with cpu.runtime.context(n_threads=1):
        serial = (A @ X).numpy()
    with cpu.runtime.context(n_threads=3):
        parallel = (A @ X).numpy()
    np.testing.assert_array_equal(serial, parallel)
    np.testing.assert_allclose(serial, z[f"{pre}.scipy"], rtol=1e-5, atol=1e-5)
    np.testing.assert_array_equal(serial, oracle.csr_matmul(z[f"{pre}.data"], z[f"{pre}.indices"],
                                                            z[f"{pre}.indptr"], z[f"{pre}.X"], shape[0]))


def test_batched_rhs(cpu):
    # reference tests/test_numerical_correctness.py:76-80 and
    # tests/test_csr_matvec.py batched matvec
    z = np.load(GOLDEN / "scipy_cases.npz")
    shape = tuple(int(v) for v in z["numcorr.shape"])
    A = cpu.csr_array((z["numcorr.data"], z["numcorr.indices"], z["numcorr.indptr"]), shape=shape)
    out = (A @ torch.from_numpy(z["numcorr.B"])).numpy()
    np.testing.assert_allclose(out, z["numcorr.dense64_B"], rtol=1e-5, atol=1e-5)
    vecs = torch.from_numpy(np.ascontiguousarray(z["numcorr.B"][:, :, 0]))
    bv = cpu.csr_batched_matvec(A, vecs).numpy()
    np.testing.assert_allclose(bv, z["numcorr.dense64_B"][:, :, 0], rtol=1e-5, atol=1e-5)


def _random_csr(rng, n_rows, n_cols, index_dtype):
    lengths = rng.integers(0, 12, n_rows)
    lengths[rng.random(n_rows) < 0.15] = 0
    lengths[rng.random(n_rows) < 0.02] = 300
    indptr = np.zeros(n_rows + 1, np.int64)
    np.cumsum(lengths, out=indptr[1:])
    nnz = int(indptr[-1])
    return rng.integers(0, n_cols, nnz).astype(index_dtype), indptr.astype(index_dtype), nnz


@pytest.mark.parametrize("vtype", ["float32", "float16", "bfloat16", "complex64"])
@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
@pytest.mark.parametrize("threads", [1, 4])
def test_native_cpu_equals_oracle(cpu, oracle, vtype, index_dtype, threads):
    rng = np.random.default_rng(13)
    n_rows, n_cols = 700, 500
    indices, indptr, nnz = _random_csr(rng, n_rows, n_cols, index_dtype)
    cplx = vtype == "complex64"
    data = storage(rng.standard_normal(nnz) + (1j * rng.standard_normal(nnz) if cplx else 0), vtype)
    x = storage(rng.standard_normal(n_cols) + (1j * rng.standard_normal(n_cols) if cplx else 0), vtype)
    X = storage(rng.standard_normal((n_cols, 6)) + (1j * rng.standard_normal((n_cols, 6)) if cplx else 0),
                vtype)
    from _util import to_torch

    A = cpu.csr_array((to_torch(data, vtype), indices, indptr), shape=(n_rows, n_cols))
    with cpu.runtime.context(n_threads=threads):
        y = to_numpy(A @ to_torch(x, vtype))
        Y = to_numpy(A @ to_torch(X, vtype))
    want_y = oracle.csr_matvec(data, indices, indptr, x, n_rows, vtype=vtype)
    want_Y = oracle.csr_matmul(data, indices, indptr, X, n_rows, vtype=vtype)
    # identical algorithms: equal values (bf16 compared as bit patterns)
    np.testing.assert_array_equal(widen(y, vtype), widen(want_y, vtype))
    np.testing.assert_array_equal(widen(Y, vtype), widen(want_Y, vtype))


def test_device_selection(ms):
    prev = ms.default_torch_device()
    try:
        assert ms.use_cpu().type == "cpu"
        assert ms.use_device("CPU").type == "cpu"
        with pytest.raises(ValueError, match="device must be"):
            ms.use_device("tpu")
        if not torch.cuda.is_available():
            with pytest.raises(RuntimeError, match="not available"):
                ms.use_gpu()
    finally:
        if prev.type == "cuda":
            ms.use_gpu(prev.index or 0)
        else:
            ms.use_cpu()


def test_runtime_context_and_info(ms, monkeypatch):
    monkeypatch.delenv("MLX_SPARSE_CPU_THREADS", raising=False)
    with ms.runtime.context(n_threads=3):
        assert ms.runtime.resolve_n_threads() == (3, "configured")
        from mlx_sparse._ext_loader import extension

        assert extension().cpu_worker_count() == 3
    with ms.runtime.context({ms.runtime.RuntimeOption.N_THREADS: 2}):
        assert ms.runtime.get("n_threads") == 2
    with pytest.raises(ValueError):
        with ms.runtime.context(n_threads=0):
            pass
    with pytest.raises(TypeError):
        with ms.runtime.context(ms.runtime.RuntimeOption.N_THREADS):
            pass
    info = ms.runtime.info()
    assert info["extension"] is True and "n_threads" in info
    caps = ms.capabilities()
    assert caps["rocm"] is True and caps["metal"] is False


def test_is_available_and_no_fallback(ms, monkeypatch):
    assert ms.is_available()
    import mlx_sparse._ext_loader as loader

    monkeypatch.setattr(loader, "_EXT", None)
    monkeypatch.setattr(loader, "_ERROR", ImportError("simulated missing build"))
    with pytest.raises(RuntimeError, match="not built"):
        loader.extension()


# -- batched right-hand sides (reference: src/sparse/csr_batched_matvec,
#    src/sparse/csr_batched_matmul) -------------------------------------------------

def _batched_want(oracle, data, indices, indptr, X, n_rows, vtype, k=None):
    """Every output summed from zero in stored order: column b of one SpMM
    over the transposed batch (vectors), or one SpMM per batch (matrices)."""
    if k is None:
        return np.ascontiguousarray(
            oracle.csr_matmul(data, indices, indptr, np.ascontiguousarray(X.T), n_rows, vtype=vtype).T)
    return np.stack([oracle.csr_matmul(data, indices, indptr, X[b], n_rows, vtype=vtype)
                     for b in range(X.shape[0])])


@pytest.mark.parametrize("vtype", ["float32", "float16", "bfloat16", "complex64"])
@pytest.mark.parametrize("threads", [1, 5])
def test_batched_native_cpu_equals_oracle(cpu, oracle, vtype, threads):
    import _capi
    from _util import storage

    rng = np.random.default_rng(21)
    n_rows, n_cols = 300, 250
    indices, indptr, nnz = _random_csr(rng, n_rows, n_cols, np.int32)
    vals = rng.standard_normal(nnz) + (1j * rng.standard_normal(nnz) if vtype == "complex64" else 0)
    data = storage(vals, vtype)
    for batch, k in ((1, None), (6, None), (3, 5), (4, 1)):
        shape = (batch, n_cols) if k is None else (batch, n_cols, k)
        xv = rng.standard_normal(shape) + (1j * rng.standard_normal(shape) if vtype == "complex64" else 0)
        X = storage(xv, vtype)
        want = _batched_want(oracle, data, indices, indptr, X, n_rows, vtype, k)
        got = np.empty_like(want)
        L, T = _capi.lib(), {"float32": 0, "float16": 1, "bfloat16": 2, "complex64": 3}[vtype]
        ptr = lambda a: a.ctypes.data
        if k is None:
            st = L.msx_csr_batched_spmv_cpu(T, 0, n_rows, n_cols, nnz, ptr(data), ptr(indices),
                                            ptr(indptr), batch, ptr(X), ptr(got), threads)
        else:
            st = L.msx_csr_batched_spmm_cpu(T, 0, n_rows, n_cols, nnz, ptr(data), ptr(indices),
                                            ptr(indptr), batch, k, ptr(X), ptr(got), threads)
        assert st == _capi.OK, _capi.last_error()
        np.testing.assert_array_equal(got.view(np.uint8), want.view(np.uint8))


def test_batched_api_on_cpu(cpu, oracle):
    rng = np.random.default_rng(22)
    indices, indptr, nnz = _random_csr(rng, 120, 90, np.int64)
    data = rng.standard_normal(nnz).astype(np.float32)
    A = cpu.csr_array((data, indices, indptr), shape=(120, 90))
    X = rng.standard_normal((2, 3, 90)).astype(np.float32)
    got = cpu.csr_batched_matvec(A, torch.from_numpy(X)).numpy()
    assert got.shape == (2, 3, 120)
    want = _batched_want(oracle, data, indices, indptr, X.reshape(6, 90), 120, "float32")
    np.testing.assert_array_equal(got.reshape(6, 120), want)
    M = rng.standard_normal((2, 2, 90, 4)).astype(np.float32)
    got = cpu.csr_batched_matmul(A, torch.from_numpy(M)).numpy()
    assert got.shape == (2, 2, 120, 4)
    np.testing.assert_array_equal(got.reshape(4, 120, 4),
                                  _batched_want(oracle, data, indices, indptr, M.reshape(4, 90, 4),
                                                120, "float32", k=4))
    np.testing.assert_array_equal((A @ torch.from_numpy(M)).numpy(), got)  # rank-4 csr_matmul
    # reference error texts (mlx_sparse/_ops.py:821-855, :1097-1115)
    with pytest.raises(ValueError, match="rank-2 or higher"):
        cpu.csr_batched_matvec(A, torch.zeros(90))
    with pytest.raises(ValueError, match="vector dimension 89"):
        cpu.csr_batched_matvec(A, torch.zeros(2, 89))
    with pytest.raises(TypeError, match="same dtype"):
        cpu.csr_batched_matvec(A, torch.zeros(2, 90, dtype=torch.float16))
    with pytest.raises(ValueError, match="rank-3 or higher"):
        cpu.csr_batched_matmul(A, torch.zeros(90, 2))
    with pytest.raises(ValueError, match="sparse dimension 91"):
        cpu.csr_batched_matmul(A, torch.zeros(2, 91, 2))
