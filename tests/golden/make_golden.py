"""Regenerate the committed golden fixtures of the CSR sparse x dense path.

Run in the build container (SciPy present; the reference checkout is read
only for its public SuiteSparse data files, never imported):

    python tests/golden/make_golden.py

Writes, next to this script:

- ``scipy_cases.npz``: inputs and SciPy products of the reference tests'
  seeded random cases (reference tests: test_csr_matvec.py:39-63 seed 456,
  test_csr_matmul.py:48-76 seed 789, test_csr_matmul.py:128-154 widths
  1..32 seeds 792+k, test_numerical_correctness.py:37-113 seeds 20260521 and
  314159), plus float64 dense products of the same inputs;
- ``suitesparse_<name>.npz``: CSR of the reference fixtures
  tests/fixtures/suitesparse/HB/{well1033,illc1033,bcsstk03}.mtx (public
  SuiteSparse matrices, read with scipy.io.mmread, duplicates summed, sorted),
  the probe vector / RHS of test_suitesparse_collection.py:159-214 and their
  SciPy products.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import scipy.io
import scipy.sparse as sp

HERE = Path(__file__).resolve().parent
MTX_DIR = Path("/root/reference/tests/fixtures/suitesparse/HB")


def _csr(m) -> dict:
    m = sp.csr_matrix(m)
    m.sum_duplicates()
    m.sort_indices()
    return {"data": m.data, "indices": m.indices.astype(np.int32),
            "indptr": m.indptr.astype(np.int32), "shape": np.array(m.shape)}


def scipy_cases() -> dict:
    out: dict[str, np.ndarray] = {}

    def put(prefix, m, **arrays):
        for k, v in _csr(m).items():
            out[f"{prefix}.{k}"] = v
        for k, v in arrays.items():
            out[f"{prefix}.{k}"] = v

    rng = np.random.default_rng(456)
    m = sp.random(96, 128, density=0.03, format="csr", dtype=np.float32, random_state=rng)
    x = rng.normal(size=(128,)).astype(np.float32)
    put("matvec456", m, x=x, scipy=(m @ x).astype(np.float32),
        dense64=m.toarray().astype(np.float64) @ x.astype(np.float64))

    rng = np.random.default_rng(789)
    m = sp.random(64, 80, density=0.04, format="csr", dtype=np.float32, random_state=rng)
    X = rng.normal(size=(80, 7)).astype(np.float32)
    put("matmul789", m, X=X, scipy=(m @ X).astype(np.float32),
        dense64=m.toarray().astype(np.float64) @ X.astype(np.float64))

    for k in (1, 2, 4, 8, 16, 32):
        rng = np.random.default_rng(792 + k)
        m = sp.random(28, 35, density=0.11, format="csr", dtype=np.float32, random_state=rng)
        m.sum_duplicates()
        m.sort_indices()
        X = rng.normal(size=(35, k)).astype(np.float32)
        put(f"widths{k}", m, X=X, scipy=(m @ X).astype(np.float32),
            dense64=m.toarray().astype(np.float64) @ X.astype(np.float64))

    rng = np.random.default_rng(20260521)
    m = sp.random(48, 64, density=0.08, format="csr", dtype=np.float32, random_state=rng)
    m.sum_duplicates()
    m.sort_indices()
    x = rng.standard_normal(64).astype(np.float32)
    X = rng.standard_normal((64, 5)).astype(np.float32)
    B = rng.standard_normal((3, 64, 4)).astype(np.float32)
    d64 = m.toarray().astype(np.float64)
    put("numcorr", m, x=x, X=X, B=B, scipy_x=(m @ x).astype(np.float32),
        scipy_X=(m @ X).astype(np.float32), dense64_x=d64 @ x, dense64_X=d64 @ X,
        dense64_B=np.einsum("ij,bjk->bik", d64, B.astype(np.float64)))

    rng = np.random.default_rng(314159)
    row = np.array([0, 0, 1, 2, 2, 2, 3], dtype=np.int32)
    col = np.array([1, 4, 2, 0, 3, 5, 4], dtype=np.int32)
    data = (rng.standard_normal(row.size) + 1j * rng.standard_normal(row.size)).astype(np.complex64)
    m = sp.coo_matrix((data, (row, col)), shape=(4, 6)).tocsr()
    x = (rng.standard_normal(6) + 1j * rng.standard_normal(6)).astype(np.complex64)
    X = (rng.standard_normal((6, 3)) + 1j * rng.standard_normal((6, 3))).astype(np.complex64)
    d128 = m.toarray().astype(np.complex128)
    put("complex", m, x=x, X=X, scipy_x=(m @ x).astype(np.complex64),
        scipy_X=(m @ X).astype(np.complex64), dense128_x=d128 @ x, dense128_X=d128 @ X)
    return out


def suitesparse(name: str) -> dict:
    m = scipy.io.mmread(MTX_DIR / f"{name}.mtx").tocsr()
    m.sum_duplicates()
    m.sort_indices()
    m = m.astype(np.float32)
    n_cols = m.shape[1]
    vector = np.linspace(-1.0, 1.0, n_cols, dtype=np.float32)
    rhs = np.stack([vector, np.cos(np.arange(n_cols, dtype=np.float32) / 5.0),
                    np.linspace(0.5, -0.25, n_cols, dtype=np.float32)], axis=1)
    d64 = m.toarray().astype(np.float64)
    out = _csr(m)
    out.update(x=vector, X=rhs, scipy_x=(m @ vector).astype(np.float32),
               scipy_X=(m @ rhs).astype(np.float32), dense64_x=d64 @ vector.astype(np.float64),
               dense64_X=d64 @ rhs.astype(np.float64))
    return out


def main() -> None:
    np.savez_compressed(HERE / "scipy_cases.npz", **scipy_cases())
    for name in ("well1033", "illc1033", "bcsstk03"):
        np.savez_compressed(HERE / f"suitesparse_{name}.npz", **suitesparse(name))
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main()
