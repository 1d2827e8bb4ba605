"""The seeded workload generators: shapes, lengths and per-row distinct,
sorted columns, including rows that hold most of the columns."""

from __future__ import annotations

import time

import numpy as np

from mlx_sparse import synthetic


def _check_rows(m, lengths=None):
    ptr = m.indptr.astype(np.int64)
    assert ptr[0] == 0 and ptr[-1] == m.nnz == m.indices.size == m.data.size
    if lengths is not None:
        np.testing.assert_array_equal(np.diff(ptr), lengths)
    key = np.repeat(np.arange(m.shape[0]), np.diff(ptr)) * m.shape[1] + m.indices
    assert np.all(np.diff(key) > 0)  # sorted, distinct within each row
    assert m.indices.min() >= 0 and m.indices.max() < m.shape[1]


def test_power_law_with_rows_of_all_columns_is_quick():
    t = time.perf_counter()
    m = synthetic.power_law(1 << 16, 2.0, 200_000, seed=0)
    assert time.perf_counter() - t < 30
    rng = np.random.default_rng(0)
    lengths = np.clip(rng.zipf(2.0, size=1 << 16), 1, 1 << 16)
    assert lengths.max() == 1 << 16  # one row holds every column
    _check_rows(m, lengths)
    np.testing.assert_allclose(m.data, 1.0 / np.repeat(lengths, lengths).astype(np.float32))


def test_random_fixed_row_and_stencils():
    m = synthetic.random_fixed_row(1 << 12, 16, seed=3)
    _check_rows(m, np.full(1 << 12, 16))
    _check_rows(synthetic.laplacian_2d(32))
    _check_rows(synthetic.poisson_3d(8))
    _check_rows(synthetic.banded(1 << 10, 8, 0.5, 10.0, seed=1))
