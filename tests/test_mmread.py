"""Matrix Market ingestion (``mmread``, ``mminfo``) and ``from_scipy``.

The reference reads its SuiteSparse fixtures with ``scipy.io.mmread`` and
canonicalises them (tests/test_suitesparse_collection.py:36-47; from_scipy,
mlx_sparse/_construct.py:854-975).  The fixtures themselves are copied under
tests/golden/mtx/ (bcsstk03, illc1033, well1033 and the right-hand sides).
The checker is SciPy's own reader: every CSR buffer must equal
``mmread(path).tocsr()`` after ``sum_duplicates`` / ``sort_indices`` and the
cast to the storage type, bit for bit; float16 against numpy's direct
float64 -> float16 rounding, bfloat16 against torch through float32.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import scipy.io as sio
import scipy.sparse as sp
import torch

import mlx_sparse as ms

MTX = Path(__file__).resolve().parent / "golden" / "mtx"
GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(autouse=True)
def _cpu(ms):
    prev = ms.default_torch_device()
    ms.use_cpu()
    yield
    if prev.type == "cuda":
        ms.use_gpu(prev.index or 0)


def _scipy_csr(path):
    S = sio.mmread(path).tocsr()
    S.sum_duplicates()
    S.sort_indices()
    return S


def _assert_csr(A, S, np_dtype=np.float32):
    assert A.shape == S.shape and A.has_canonical_format
    np.testing.assert_array_equal(A.indptr.numpy(), S.indptr)
    np.testing.assert_array_equal(A.indices.numpy(), S.indices)
    want = np.asarray(S.data).astype(np_dtype)
    assert A.data.numpy().tobytes() == want.tobytes()


@pytest.mark.parametrize("name", ["bcsstk03", "well1033", "illc1033"])
@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
def test_suitesparse_fixtures_equal_scipy(name, index_dtype):
    A = ms.mmread(MTX / f"{name}.mtx", index_dtype=index_dtype)
    assert A.indices.dtype == index_dtype
    _assert_csr(A, _scipy_csr(MTX / f"{name}.mtx"))
    # and the golden arrays made from the same files
    z = np.load(GOLDEN / f"suitesparse_{name}.npz", allow_pickle=False)
    keys = [k for k in z.files if k.endswith(".indptr")]
    if keys:
        prefix = keys[0][: -len(".indptr")]
        np.testing.assert_array_equal(A.indptr.numpy(), z[f"{prefix}.indptr"])
        np.testing.assert_array_equal(A.indices.numpy(), z[f"{prefix}.indices"])


def test_mminfo_and_right_hand_sides():
    for name in ("bcsstk03", "well1033", "illc1033", "well1033_b"):
        assert ms.mminfo(MTX / f"{name}.mtx") == sio.mminfo(MTX / f"{name}.mtx")
    b = ms.mmread(MTX / "well1033_b.mtx")
    want = np.asarray(sio.mmread(MTX / "well1033_b.mtx"), dtype=np.float32)
    assert b.shape == (1033, 1) and b.numpy().tobytes() == want.tobytes()


def _write(tmp_path, name, M, **kw):
    p = tmp_path / f"{name}.mtx"
    sio.mmwrite(p, M, **kw)
    return p


@pytest.mark.parametrize("symmetry", ["general", "symmetric", "skew-symmetric"])
def test_symmetry_kinds(tmp_path, symmetry):
    rng = np.random.default_rng(1)
    n = 40
    M = sp.random(n, n, density=0.1, random_state=2, format="coo").toarray()
    if symmetry == "symmetric":
        M = M + M.T
    elif symmetry == "skew-symmetric":
        M = M - M.T
    p = _write(tmp_path, symmetry, sp.coo_matrix(M), symmetry=symmetry)
    assert ms.mminfo(p)[5] == symmetry
    _assert_csr(ms.mmread(p), _scipy_csr(p))
    assert rng is not None


def test_hermitian_complex_pattern_integer(tmp_path):
    n = 30
    R = sp.random(n, n, density=0.15, random_state=3).toarray()
    I = sp.random(n, n, density=0.15, random_state=4).toarray()
    H = (R + 1j * I)
    H = np.triu(H, 1) + np.triu(H, 1).conj().T + np.diag(np.arange(n, dtype=float))
    p = _write(tmp_path, "herm", sp.coo_matrix(H), symmetry="hermitian")
    A = ms.mmread(p)
    assert A.dtype == torch.complex64
    _assert_csr(A, _scipy_csr(p), np.complex64)
    with pytest.raises(TypeError, match="complex64"):
        ms.mmread(p, dtype=torch.float32)
    P = sp.coo_matrix((np.ones(5), ([0, 1, 2, 3, 4], [4, 3, 2, 1, 0])), shape=(5, 5))
    p = _write(tmp_path, "pattern", P, field="pattern")
    _assert_csr(ms.mmread(p), _scipy_csr(p))
    Z = sp.coo_matrix((np.array([3, -7, 12]), ([0, 2, 1], [1, 0, 2])), shape=(3, 3))
    p = _write(tmp_path, "int", Z, field="integer")
    assert ms.mminfo(p)[4] == "integer"
    _assert_csr(ms.mmread(p), _scipy_csr(p))


def test_duplicates_comments_and_notation(tmp_path):
    text = """%%MatrixMarket matrix coordinate real general
% a comment
%

4 5 7
1 1 1.5e0
2 3 -2.25
1 1 0.25
4 5 1E-3
3 2 7
2 3 0.125
4 1 -0
"""
    p = tmp_path / "dups.mtx"
    p.write_text(text)
    _assert_csr(ms.mmread(p), _scipy_csr(p))
    A = ms.mmread(p)
    # blank and comment lines inside the data section are skipped (SciPy's
    # reader refuses them): the same matrix
    loose = tmp_path / "loose.mtx"
    loose.write_text(text.replace("3 2 7\n", "\n3 2 7\n% interleaved\n"))
    L = ms.mmread(loose)
    assert torch.equal(L.indptr, A.indptr) and torch.equal(L.data, A.data)
    assert A.nnz == 5 and A.data[0].item() == 1.75
    assert A.data.numpy()[A.indptr[3]].tobytes() == np.float32(-0.0).tobytes()
    # a leading '+' (C scanf accepts it; SciPy's reader does not)
    p.write_text(text.replace("1 1 0.25", "1 1 +0.25"))
    assert ms.mmread(p).data[0].item() == 1.75


def test_array_files(tmp_path):
    rng = np.random.default_rng(5)
    D = rng.standard_normal((7, 3))
    p = _write(tmp_path, "dense", D)
    assert ms.mminfo(p)[3] == "array"
    got = ms.mmread(p)
    assert got.shape == (7, 3) and got.numpy().tobytes() == D.astype(np.float32).tobytes()
    S = rng.standard_normal((5, 5))
    S = S + S.T
    p = _write(tmp_path, "dense_sym", S, symmetry="symmetric")
    np.testing.assert_array_equal(ms.mmread(p).numpy(), np.asarray(sio.mmread(p), np.float32))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_low_precision_rounding(tmp_path, dtype):
    rng = np.random.default_rng(6)
    n = 4000
    # wide range: subnormal halves, ties, overflow to inf for float16
    vals = rng.standard_normal(n) * np.exp2(rng.integers(-30, 20, n))
    vals[:4] = [65520.0, 65519.99, 2.0 ** -25, 3 * 2.0 ** -26]
    rows = np.arange(n) % 97
    cols = np.arange(n) // 97
    M = sp.coo_matrix((vals, (rows, cols)), shape=(97, n // 97 + 1))
    p = _write(tmp_path, "round", M, precision=17)
    A = ms.mmread(p, dtype=dtype)
    S = _scipy_csr(p)
    np.testing.assert_array_equal(A.indices.numpy(), S.indices)
    if dtype == torch.float16:
        want = torch.from_numpy(S.data.astype(np.float16))
    else:
        want = torch.from_numpy(S.data.astype(np.float32)).to(torch.bfloat16)
    assert torch.equal(A.data.view(torch.int16), want.view(torch.int16))


def test_large_file_multithreaded(tmp_path):
    rng = np.random.default_rng(7)
    n, m = 50_000, 400_000
    M = sp.coo_matrix((rng.standard_normal(m), (rng.integers(0, n, m), rng.integers(0, n, m))),
                      shape=(n, n))
    p = _write(tmp_path, "big", M)
    for threads in (1, 8):
        _assert_csr(ms.mmread(p, n_threads=threads), _scipy_csr(p))


def test_errors(tmp_path):
    with pytest.raises(ValueError, match="cannot read"):
        ms.mmread(tmp_path / "missing.mtx")
    bad = tmp_path / "bad.mtx"
    bad.write_text("%%MatrixMarket tensor coordinate real general\n2 2 1\n1 1 1\n")
    with pytest.raises(ValueError, match="header"):
        ms.mmread(bad)
    bad.write_text("%%MatrixMarket matrix coordinate real general\n2 2 2\n1 1 1\n")
    with pytest.raises(ValueError, match="promises 2"):
        ms.mmread(bad)
    bad.write_text("%%MatrixMarket matrix coordinate real general\n2 2 1\n3 1 1\n")
    with pytest.raises(ValueError, match="bad data line"):
        ms.mmread(bad)
    bad.write_text("%%MatrixMarket matrix coordinate real symmetric\n2 3 1\n1 1 1\n")
    with pytest.raises(ValueError, match="square"):
        ms.mmread(bad)


def test_from_scipy():
    S = sp.csr_matrix(np.array([[0, 2.5, 0], [1.0, 0, -3.0]]))
    A = ms.from_scipy(S)
    assert A.dtype == torch.float32 and A.has_canonical_format and A.shape == (2, 3)
    np.testing.assert_array_equal(A.todense().numpy(), S.toarray().astype(np.float32))
    assert ms.from_scipy(S, dtype=torch.bfloat16).dtype == torch.bfloat16
    assert ms.from_scipy(S, dtype=torch.float16).dtype == torch.float16
    assert ms.from_scipy(S.astype(np.complex128)).dtype == torch.complex64
    assert ms.from_scipy(S, index_dtype=torch.int64).indices.dtype == torch.int64
    dup = sp.coo_matrix((np.ones(3), ([0, 0, 1], [1, 1, 0])), shape=(2, 2))
    assert ms.from_scipy(dup).nnz == 2
    with pytest.raises(TypeError, match="scipy.sparse"):
        ms.from_scipy(np.eye(2))
    with pytest.raises(ValueError, match="format"):
        ms.from_scipy(S, format="csc")


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["bcsstk03", "well1033", "illc1033"])
def test_fixture_spmv_on_gpu(ms, oracle, name):
    """The SuiteSparse fixtures through mmread, then ``A @ x`` on the GPU,
    equal to the oracle bit for bit (short f32 rows)."""
    ms.use_gpu()
    try:
        A = ms.mmread(MTX / f"{name}.mtx")
        assert A.data.device.type == "cuda"
        x = torch.linspace(-1, 1, A.shape[1], device="cuda")
        y = (A @ x).cpu().numpy()
    finally:
        ms.use_cpu()
    want = oracle.csr_matvec(A.data.cpu().numpy(), A.indices.cpu().numpy(),
                             A.indptr.cpu().numpy(), x.cpu().numpy(), A.shape[0])
    assert y.tobytes() == want.tobytes()
