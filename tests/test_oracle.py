"""Pins the CPU oracle (oracle/csr_oracle.c) before it is trusted as the
checker of the HIP path.

Each check is chosen so that a plausible mistake in the oracle fails it:
reference known-answer tests, SciPy products of the reference tests' seeded
inputs and SuiteSparse fixtures (tests/golden, made by make_golden.py),
closed forms of stencil matrices, float64 brute force, the float16/bfloat16
rounding against numpy and torch, accumulation-width probes, and the
worker-range rule against a naive re-derivation.
"""

from __future__ import annotations

import os
from pathlib import Path

import numpy as np
import pytest
import torch

from _util import storage, widen

GOLDEN = Path(__file__).resolve().parent / "golden"


def _golden(name):
    return np.load(GOLDEN / name, allow_pickle=False)


def _case(z, prefix):
    return (z[f"{prefix}.data"], z[f"{prefix}.indices"], z[f"{prefix}.indptr"],
            tuple(int(v) for v in z[f"{prefix}.shape"]))


# -- reference known-answer tests ---------------------------------------------

KAT_DATA = np.array([2.0, -1.0, 4.0, 5.0], np.float32)
KAT_IND = np.array([0, 2, 1, 3], np.int32)
KAT_PTR = np.array([0, 2, 2, 4], np.int32)


def test_kat_matvec(oracle):
    # reference tests/test_csr_matvec.py:25-36
    y = oracle.csr_matvec(KAT_DATA, KAT_IND, KAT_PTR, np.array([3, 10, 7, -2], np.float32), 3)
    np.testing.assert_array_equal(y, np.array([-1.0, 0.0, 30.0], np.float32))


def test_kat_matmul(oracle):
    # reference tests/test_csr_matmul.py:25-45
    X = np.array([[3, 1], [10, -2], [7, 4], [-2, 6]], np.float32)
    Y = oracle.csr_matmul(KAT_DATA, KAT_IND, KAT_PTR, X, 3)
    np.testing.assert_array_equal(Y, np.array([[-1, -2], [0, 0], [30, 22]], np.float32))


def test_kat_int64_unsorted_serial_parallel(oracle):
    import scipy.sparse as scipy

    # reference tests/test_csr_matvec.py:100-133
    data = np.array([2.0, -1.0, 0.5, 3.0, -4.0, 1.25, 2.5, -0.75, 4.0], np.float32)
    ind = np.array([0, 3, 1, 2, 5, 0, 4, 1, 5], np.int64)
    ptr = np.array([0, 2, 2, 5, 6, 9], np.int64)
    x = np.array([1.0, -2.0, 0.5, 3.0, -1.5, 2.5], np.float32)
    expected = scipy.csr_matrix((data, ind.astype(np.int32), ptr.astype(np.int32)), shape=(5, 6)) @ x
    serial = oracle.csr_matvec(data, ind, ptr, x, 5, n_threads=1)
    par = oracle.csr_matvec(data, ind, ptr, x, 5, n_threads=3)
    np.testing.assert_allclose(serial, expected, rtol=1e-5, atol=1e-5)
    np.testing.assert_array_equal(serial, par)


@pytest.mark.parametrize("vtype", ["float16", "float32", "complex64"])
def test_kat_dtypes(oracle, vtype):
    # reference tests/test_dtypes.py:24-61
    vals = np.array([2.0, -1.0, 4.0, 5.0])
    x = np.array([3.0, 10.0, 7.0, -2.0])
    if vtype == "complex64":
        vals = vals + np.array([1j, -2j, 0.5j, 3j])
        x = x + np.array([-1j, 2j, 0j, -0.5j])
    v, xs = storage(vals, vtype), storage(x, vtype)
    want = np.array([v[0] * xs[0] + v[1] * xs[2], 0, v[2] * xs[1] + v[3] * xs[3]])
    got = oracle.csr_matvec(v, KAT_IND, KAT_PTR, xs, 3, vtype=vtype)
    tol = 5e-3 if vtype == "float16" else 1e-5
    np.testing.assert_allclose(widen(got, vtype), want.astype(np.complex128 if vtype == "complex64" else np.float64),
                               rtol=tol, atol=tol)


def test_kat_bfloat16(oracle):
    # reference tests/test_dtypes.py:64-77: [2, -1] . [3, 7] = -1 in bfloat16
    d = storage(np.array([2.0, -1.0]), "bfloat16")
    x = storage(np.array([3.0, 7.0]), "bfloat16")
    y = oracle.csr_matvec(d, np.array([0, 1], np.int32), np.array([0, 2], np.int32), x, 1,
                          vtype="bfloat16")
    assert widen(y, "bfloat16")[0] == -1.0


@pytest.mark.parametrize("vtype,tol", [("float16", 5e-3), ("bfloat16", 2e-2)])
def test_kat_low_precision_matmul(oracle, vtype, tol):
    # reference tests/test_dtypes.py:80-110
    d = storage(np.array([2.0, -1.0, 4.0]), vtype)
    X = storage(np.array([[3.0, 1.0], [10.0, -2.0], [7.0, 4.0]]), vtype)
    Y = oracle.csr_matmul(d, np.array([0, 2, 1], np.int32), np.array([0, 2, 3], np.int32), X, 2,
                          vtype=vtype)
    np.testing.assert_allclose(widen(Y, vtype), [[-1.0, -2.0], [40.0, -8.0]], rtol=tol, atol=tol)


# -- SciPy products of the reference tests' seeded inputs --------------------

def test_scipy_matvec_seed456(oracle):
    z = _golden("scipy_cases.npz")
    d, i, p, shape = _case(z, "matvec456")
    y = oracle.csr_matvec(d, i, p, z["matvec456.x"], shape[0])
    # SciPy's loop is the same sequential float32 sum from zero
    np.testing.assert_array_equal(y, z["matvec456.scipy"])
    np.testing.assert_allclose(y, z["matvec456.dense64"], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("prefix", ["matmul789", "widths1", "widths2", "widths4", "widths8",
                                    "widths16", "widths32"])
def test_scipy_matmul(oracle, prefix):
    z = _golden("scipy_cases.npz")
    d, i, p, shape = _case(z, prefix)
    Y = oracle.csr_matmul(d, i, p, z[f"{prefix}.X"], shape[0])
    np.testing.assert_allclose(Y, z[f"{prefix}.scipy"], rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(Y, z[f"{prefix}.dense64"], rtol=1e-5, atol=1e-5)
    # column c of the SpMM equals the SpMV of column c
    X = z[f"{prefix}.X"]
    for c in range(X.shape[1]):
        np.testing.assert_array_equal(Y[:, c], oracle.csr_matvec(d, i, p, X[:, c].copy(), shape[0]))
    Y3 = oracle.csr_matmul(d, i, p, X, shape[0], n_threads=3)
    np.testing.assert_array_equal(Y, Y3)


def test_numerical_correctness_seed20260521(oracle):
    # reference tests/test_numerical_correctness.py:37-80
    z = _golden("scipy_cases.npz")
    d, i, p, shape = _case(z, "numcorr")
    y = oracle.csr_matvec(d, i, p, z["numcorr.x"], shape[0])
    np.testing.assert_allclose(y, z["numcorr.dense64_x"], rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(y, z["numcorr.scipy_x"], rtol=1e-5, atol=1e-5)
    Y = oracle.csr_matmul(d, i, p, z["numcorr.X"], shape[0])
    np.testing.assert_allclose(Y, z["numcorr.dense64_X"], rtol=1e-5, atol=1e-5)


def test_complex_seed314159(oracle):
    # reference tests/test_numerical_correctness.py:83-113
    z = _golden("scipy_cases.npz")
    d, i, p, shape = _case(z, "complex")
    y = oracle.csr_matvec(d, i, p, z["complex.x"], shape[0])
    np.testing.assert_allclose(y, z["complex.dense128_x"], rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(y, z["complex.scipy_x"], rtol=1e-5, atol=1e-5)
    Y = oracle.csr_matmul(d, i, p, z["complex.X"], shape[0])
    np.testing.assert_allclose(Y, z["complex.dense128_X"], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("name,rtol,atol", [("well1033", 2e-5, 2e-5), ("illc1033", 2e-5, 2e-5),
                                            ("bcsstk03", 2e-5, 3.0e6)])
def test_suitesparse(oracle, name, rtol, atol):
    # reference tests/test_suitesparse_collection.py:27-32,159-214
    z = _golden(f"suitesparse_{name}.npz")
    shape = tuple(int(v) for v in z["shape"])
    y = oracle.csr_matvec(z["data"], z["indices"], z["indptr"], z["x"], shape[0])
    np.testing.assert_array_equal(y, z["scipy_x"])
    np.testing.assert_allclose(y, z["dense64_x"], rtol=rtol, atol=atol)
    Y = oracle.csr_matmul(z["data"], z["indices"], z["indptr"], z["X"], shape[0])
    np.testing.assert_allclose(Y, z["scipy_X"], rtol=rtol, atol=atol)
    np.testing.assert_allclose(Y, z["dense64_X"], rtol=rtol, atol=atol)


# -- closed forms ---------------------------------------------------------------

def test_laplacian_closed_forms(oracle):
    from mlx_sparse import synthetic

    g = 64
    m = synthetic.laplacian_2d(g)
    ones = np.ones(m.shape[1], np.float32)
    y = oracle.csr_matvec(m.data, m.indices, m.indptr, ones, m.shape[0]).reshape(g, g)
    want = np.zeros((g, g), np.float32)
    want[0, :] += 1
    want[-1, :] += 1
    want[:, 0] += 1
    want[:, -1] += 1
    np.testing.assert_array_equal(y, want)  # 4 - (#neighbours): 0 inside, 1 edges, 2 corners
    # discrete Laplacian of a linear field vanishes in the interior
    ii, jj = np.meshgrid(np.arange(g), np.arange(g), indexing="ij")
    lin = (3 * ii + 5 * jj).astype(np.float32).reshape(-1)
    y = oracle.csr_matvec(m.data, m.indices, m.indptr, lin, m.shape[0]).reshape(g, g)
    np.testing.assert_array_equal(y[1:-1, 1:-1], 0)


def test_poisson_closed_form(oracle):
    from mlx_sparse import synthetic

    g = 16
    m = synthetic.poisson_3d(g)
    y = oracle.csr_matvec(m.data, m.indices, m.indptr, np.ones(m.shape[1], np.float32),
                          m.shape[0]).reshape(g, g, g)
    k, i, j = np.meshgrid(np.arange(g), np.arange(g), np.arange(g), indexing="ij")
    boundary = ((k == 0) | (k == g - 1)).astype(int) + ((i == 0) | (i == g - 1)).astype(int) \
        + ((j == 0) | (j == g - 1)).astype(int)
    np.testing.assert_array_equal(y, boundary.astype(np.float32))
    # SpMM with X = [1, 2*1]: both columns exact
    X = np.stack([np.ones(m.shape[1]), 2 * np.ones(m.shape[1])], 1).astype(np.float32)
    Y = oracle.csr_matmul(m.data, m.indices, m.indptr, X, m.shape[0])
    np.testing.assert_array_equal(Y[:, 1], 2 * Y[:, 0])


def test_power_law_row_normalised(oracle):
    from mlx_sparse import synthetic

    m = synthetic.power_law(n=4096, max_len=3000, seed=1)
    y = oracle.csr_matvec(m.data, m.indices, m.indptr, np.ones(m.shape[1], np.float32), m.shape[0])
    lengths = np.diff(m.indptr)
    # sum of L copies of fl(1/L): within L ulps of 1
    assert np.all(np.abs(y.astype(np.float64) - 1.0) <= lengths * 2.0**-23)


# -- float64 brute force on random inputs (empty rows, duplicates, unsorted) ----

def _random_csr(rng, n_rows, n_cols, density, index_dtype, dup=True):
    lengths = rng.binomial(n_cols, density, size=n_rows)
    lengths[rng.random(n_rows) < 0.2] = 0  # empty rows
    indptr = np.zeros(n_rows + 1, np.int64)
    np.cumsum(lengths, out=indptr[1:])
    nnz = int(indptr[-1])
    indices = rng.integers(0, n_cols, nnz)  # unsorted, duplicates allowed
    return indices.astype(index_dtype), indptr.astype(index_dtype), nnz


@pytest.mark.parametrize("vtype", ["float32", "float16", "bfloat16", "complex64"])
@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_brute_force(oracle, vtype, index_dtype):
    rng = np.random.default_rng(7)
    n_rows, n_cols = 57, 41
    ind, ptr, nnz = _random_csr(rng, n_rows, n_cols, 0.3, index_dtype)
    vals = rng.standard_normal(nnz) + (1j * rng.standard_normal(nnz) if vtype == "complex64" else 0)
    x = rng.standard_normal(n_cols) + (1j * rng.standard_normal(n_cols) if vtype == "complex64" else 0)
    X = rng.standard_normal((n_cols, 5)) + (1j * rng.standard_normal((n_cols, 5)) if vtype == "complex64" else 0)
    d, xs, Xs = storage(vals, vtype), storage(x, vtype), storage(X, vtype)
    dense = np.zeros((n_rows, n_cols), np.complex128 if vtype == "complex64" else np.float64)
    rows = np.repeat(np.arange(n_rows), np.diff(ptr.astype(np.int64)))
    np.add.at(dense, (rows, ind.astype(np.int64)), widen(d, vtype))
    tol = 1e-2 if vtype in ("float16", "bfloat16") else 1e-5
    y = oracle.csr_matvec(d, ind, ptr, xs, n_rows, vtype=vtype)
    want = dense @ widen(xs, vtype)
    scale = np.abs(dense) @ np.abs(widen(xs, vtype))
    assert np.all(np.abs(widen(y, vtype) - want) <= tol * scale + 1e-30)
    Y = oracle.csr_matmul(d, ind, ptr, Xs, n_rows, vtype=vtype)
    want = dense @ widen(Xs, vtype)
    scale = np.abs(dense) @ np.abs(widen(Xs, vtype))
    assert np.all(np.abs(widen(Y, vtype) - want) <= tol * scale + 1e-30)
    # empty rows give exact zeros
    empty = np.diff(ptr.astype(np.int64)) == 0
    assert np.all(widen(y, vtype)[empty] == 0)


# -- accumulation width: low-precision values sum in float32 ---------------------

@pytest.mark.parametrize("vtype", ["float16", "bfloat16"])
def test_low_precision_accumulates_in_float32(oracle, vtype):
    # 1024 + 1 + 1 + ... (512 ones): in float32 the sum is 1536 exactly; a
    # storage-type accumulator loses every +1 once the spacing exceeds 2
    # (bfloat16 above 256, float16 above 2048).  1536 is exact in both types.
    n = 513
    vals = np.ones(n)
    vals[0] = 1024.0
    d = storage(vals, vtype)
    x = storage(np.ones(n), vtype)
    y = oracle.csr_matvec(d, np.arange(n, dtype=np.int32), np.array([0, n], np.int32), x, 1,
                          vtype=vtype)
    assert widen(y, vtype)[0] == 1536.0
    # products are formed in float32 before the sum: 3 * (1/3 rounded) terms
    # of a value whose product is not representable in the storage type
    third = storage(np.array([1.0 / 3.0]), vtype)
    three = storage(np.array([3.0]), vtype)
    y = oracle.csr_matvec(np.repeat(third, 3), np.zeros(3, np.int32), np.array([0, 3], np.int32),
                          three, 1, vtype=vtype)
    p = widen(third, vtype)[0] * 3.0  # exact in float64
    s = np.float32(np.float32(np.float32(p) + np.float32(p)) + np.float32(p))
    want = storage(np.array([s], np.float32), vtype)
    assert widen(y, vtype)[0] == widen(want, vtype)[0]


# -- rounding of the storage types ---------------------------------------------

def _probe_floats(rng, n=1 << 20):
    bits = rng.integers(0, 2**32, size=n, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    f = f[np.isfinite(f)]
    # halfway cases of float16 and bfloat16 and subnormal / overflow edges
    ties16 = (np.arange(0, 65504, 0.5, dtype=np.float64)[::97] + 2**-25).astype(np.float32)
    edges = np.array([0.0, -0.0, 2**-24, 2**-25, 3 * 2**-26, 65504, 65519.99, 65520, 1e-45,
                      np.finfo(np.float32).max, np.finfo(np.float32).tiny], np.float32)
    return np.concatenate([f, ties16, edges, -edges])


def test_f16_rounding_matches_numpy(oracle):
    f = _probe_floats(np.random.default_rng(11))
    got = oracle.f32_to_f16_bits(f)
    want = f.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, want)
    every = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    wide = oracle.f16_bits_to_f32(every)
    ref = every.view(np.float16).astype(np.float32)
    np.testing.assert_array_equal(np.isnan(wide), np.isnan(ref))
    ok = ~np.isnan(ref)
    np.testing.assert_array_equal(wide[ok].view(np.uint32), ref[ok].view(np.uint32))


def test_bf16_rounding_matches_torch(oracle):
    f = _probe_floats(np.random.default_rng(12))
    got = oracle.f32_to_bf16_bits(f)
    want = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got, want)
    every = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    wide = oracle.bf16_bits_to_f32(every)
    ref = torch.from_numpy(every.view(np.int16)).view(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(np.isnan(wide), np.isnan(ref))
    ok = ~np.isnan(ref)
    np.testing.assert_array_equal(wide[ok].view(np.uint32), ref[ok].view(np.uint32))


# -- complex product structure ----------------------------------------------------

def test_complex_splits_into_real_spmvs(oracle):
    rng = np.random.default_rng(5)
    ind, ptr, nnz = _random_csr(rng, 40, 30, 0.4, np.int32)
    re, im = rng.standard_normal(nnz).astype(np.float32), rng.standard_normal(nnz).astype(np.float32)
    x = rng.standard_normal(30).astype(np.float32)
    yc = oracle.csr_matvec((re + 1j * im).astype(np.complex64), ind, ptr, x.astype(np.complex64), 40)
    # (a + ib) * (x + 0i) = (a x - b 0) + i (a 0 + b x): exact splits
    np.testing.assert_array_equal(yc.real, oracle.csr_matvec(re, ind, ptr, x, 40))
    np.testing.assert_array_equal(yc.imag, oracle.csr_matvec(im, ind, ptr, x, 40))


# -- worker ranges and count ------------------------------------------------------

def _naive_ranges(work, parts):
    """The range rule re-derived with plain loops (reference
    cpu_parallel.h:134-164, cpu_parallel.cpp:183-253)."""
    n = len(work)
    if n == 0:
        return []
    if parts <= 1:
        return [(0, n)]
    w = [max(0, int(v)) for v in work]

    def equal(count):
        out = []
        for p in range(count):
            b, e = p * n // count, (p + 1) * n // count
            if b < e:
                out.append((b, e))
        return out

    if all(v == w[0] for v in w):
        return equal(parts)
    if parts >= n:
        return equal(parts)
    total = sum(w)
    if total <= 0:
        return equal(parts)
    out, begin = [], 0
    for part in range(parts):
        if begin >= n:
            break
        left = parts - part
        if left == 1:
            out.append((begin, n))
            break
        done = sum(w[:begin])
        target = done + -(-(total - done) // left)
        end, acc = begin + 1, done + w[begin]
        while end < n and acc < target:
            acc += w[end]
            end += 1
        end = min(max(end, begin + 1), n - (left - 1))
        out.append((begin, end))
        begin = end
    return out


@pytest.mark.parametrize("seed", range(6))
def test_cpu_ranges_match_naive_rule(oracle, ms, seed):
    from mlx_sparse._ext_loader import extension

    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 200))
    work = rng.integers(0, 50, n)
    if seed == 0:
        work[:] = 7  # balanced: equal ranges
    if seed == 1:
        work[: n // 2] = 0
    for parts in (1, 2, 3, 5, 8, 300):
        want = _naive_ranges(list(work), parts)
        assert oracle.cpu_ranges(work, parts) == want
        assert [tuple(r) for r in extension().cpu_ranges(list(map(int, work)), parts)] == want


@pytest.mark.parametrize("env,want", [
    ({"MLX_SPARSE_CPU_THREADS": "3"}, 3),
    ({"MLX_SPARSE_CPU_THREADS": "", "MLX_SPARSE_N_THREADS": "6"}, 6),
    ({"OMP_NUM_THREADS": "5"}, 5),
    ({"OMP_NUM_THREADS": "4,2"}, 4),
    ({"OMP_NUM_THREADS": "x", "SLURM_CPUS_PER_TASK": "9"}, 9),
])
def test_worker_count_resolution(oracle, ms, monkeypatch, env, want):
    from mlx_sparse._ext_loader import extension

    for name in ("MLX_SPARSE_CPU_THREADS", "MLX_SPARSE_N_THREADS", "OMP_NUM_THREADS",
                 "SLURM_CPUS_PER_TASK", "PBS_NP", "LSB_DJOB_NUMPROC", "NSLOTS"):
        monkeypatch.delenv(name, raising=False)
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    assert oracle.cpu_worker_count() == want
    assert extension().cpu_worker_count() == want


def test_worker_count_affinity_default(oracle, ms, monkeypatch):
    from mlx_sparse._ext_loader import extension

    for name in ("MLX_SPARSE_CPU_THREADS", "MLX_SPARSE_N_THREADS", "OMP_NUM_THREADS",
                 "SLURM_CPUS_PER_TASK", "PBS_NP", "LSB_DJOB_NUMPROC", "NSLOTS"):
        monkeypatch.delenv(name, raising=False)
    assert oracle.cpu_worker_count() == len(os.sched_getaffinity(0))
    assert extension().cpu_worker_count() == len(os.sched_getaffinity(0))
