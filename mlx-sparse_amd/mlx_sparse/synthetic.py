"""Seeded synthetic CSR matrices of the benchmark configurations.

Each generator returns a :class:`Matrix` of numpy arrays (canonical CSR:
sorted, duplicate-free columns) so the same inputs feed the GPU path, the
CPU path and the test oracle.  Sizes are parameters, so tests build the same
structures at small sizes.

- ``laplacian_2d(g)``: 5-point Laplacian on a g x g grid, diag 4, off -1;
- ``random_fixed_row(n, per_row)``: ``per_row`` columns per row drawn
  uniformly without replacement, values N(0, 1);
- ``power_law(n, alpha, max_len)``: row lengths ~ Zipf(alpha) clipped to
  [1, max_len], columns uniform without replacement, values 1/row_length;
- ``poisson_3d(g)``: 7-point Poisson on a g^3 grid, diag 6, off -1;
- ``banded(n, half_band, fill, shift)``: band |i-j| <= half_band, diagonal
  always stored, off-diagonals kept with probability ``fill``, values
  N(0, 1) plus ``shift`` on the diagonal.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass
class Matrix:
    name: str
    data: np.ndarray  # float32 (or complex64)
    indices: np.ndarray
    indptr: np.ndarray
    shape: tuple[int, int]

    @property
    def nnz(self) -> int:
        return int(self.data.shape[0])


def _indptr_from_lengths(lengths: np.ndarray, dtype) -> np.ndarray:
    indptr = np.zeros(lengths.shape[0] + 1, dtype=np.int64)
    np.cumsum(lengths, out=indptr[1:])
    return indptr.astype(dtype)


def _stencil(offsets_valid: list[tuple[np.ndarray, np.ndarray, float]], n: int, index_dtype):
    """Assemble sorted CSR rows from per-offset (column, valid) arrays given
    in increasing column-offset order."""
    valid = np.stack([v for _, v, _ in offsets_valid], axis=1)
    cols = np.stack([c for c, _, _ in offsets_valid], axis=1)
    vals = np.broadcast_to(np.array([w for _, _, w in offsets_valid], dtype=np.float32), cols.shape)
    lengths = valid.sum(axis=1)
    indices = cols[valid].astype(index_dtype)
    data = np.ascontiguousarray(vals[valid], dtype=np.float32)
    return data, indices, _indptr_from_lengths(lengths, index_dtype)


def laplacian_2d(g: int = 1024, index_dtype=np.int32) -> Matrix:
    n = g * g
    idx = np.arange(n, dtype=np.int64)
    i, j = idx // g, idx % g
    parts = [
        (idx - g, i > 0, -1.0),
        (idx - 1, j > 0, -1.0),
        (idx, np.ones(n, bool), 4.0),
        (idx + 1, j < g - 1, -1.0),
        (idx + g, i < g - 1, -1.0),
    ]
    data, indices, indptr = _stencil(parts, n, index_dtype)
    return Matrix(f"laplacian2d_{g}", data, indices, indptr, (n, n))


def poisson_3d(g: int = 128, index_dtype=np.int32) -> Matrix:
    n = g * g * g
    idx = np.arange(n, dtype=np.int64)
    k, rem = idx // (g * g), idx % (g * g)
    i, j = rem // g, rem % g
    parts = [
        (idx - g * g, k > 0, -1.0),
        (idx - g, i > 0, -1.0),
        (idx - 1, j > 0, -1.0),
        (idx, np.ones(n, bool), 6.0),
        (idx + 1, j < g - 1, -1.0),
        (idx + g, i < g - 1, -1.0),
        (idx + g * g, k < g - 1, -1.0),
    ]
    data, indices, indptr = _stencil(parts, n, index_dtype)
    return Matrix(f"poisson3d_{g}", data, indices, indptr, (n, n))


def _distinct_sorted_columns(lengths: np.ndarray, n_cols: int, rng) -> tuple[np.ndarray, np.ndarray]:
    """Per-row distinct sorted columns, uniform without replacement: draw with
    replacement, drop duplicates, redraw the shortfall until none is left."""
    n = lengths.shape[0]
    # Rows holding more than an eighth of the columns are drawn directly
    # without replacement: redrawing duplicates would need many rounds there.
    wide = np.flatnonzero(lengths > n_cols // 8)
    if wide.size:
        narrow = lengths.copy()
        narrow[wide] = 0
        rows, cols = _distinct_sorted_columns(narrow, n_cols, rng)
        extra = [np.sort(rng.choice(n_cols, size=int(lengths[r]), replace=False)) for r in wide]
        rows = np.concatenate([rows] + [np.full(e.size, r, np.int64) for r, e in zip(wide, extra)])
        cols = np.concatenate([cols] + [e.astype(np.int64) for e in extra])
        order = np.argsort(rows * n_cols + cols, kind="stable")
        return rows[order], cols[order]
    rows = np.repeat(np.arange(n, dtype=np.int64), lengths)
    cols = rng.integers(0, n_cols, size=rows.shape[0], dtype=np.int64)
    while True:
        key = rows * n_cols + cols
        key = np.unique(key)
        rows = key // n_cols
        cols = key % n_cols
        have = np.bincount(rows, minlength=n)
        short = lengths - have
        if not short.any():
            break
        extra_rows = np.repeat(np.arange(n, dtype=np.int64), short)
        extra_cols = rng.integers(0, n_cols, size=extra_rows.shape[0], dtype=np.int64)
        rows = np.concatenate([rows, extra_rows])
        cols = np.concatenate([cols, extra_cols])
    return rows, cols


def random_fixed_row(n: int = 4_194_304, per_row: int = 16, seed: int = 0,
                     index_dtype=np.int32) -> Matrix:
    rng = np.random.default_rng(seed)
    if n >= 65536:
        # rows drawn as one (n, per_row) block, sorted in place; rows with a
        # repeated column are redrawn (rare: ~per_row^2 / 2n per row)
        cols = rng.integers(0, n, size=(n, per_row), dtype=np.int64).astype(index_dtype)
        cols.sort(axis=1)
        while True:
            bad = np.nonzero((cols[:, 1:] == cols[:, :-1]).any(axis=1))[0]
            if bad.size == 0:
                break
            redraw = rng.integers(0, n, size=(bad.size, per_row), dtype=np.int64).astype(index_dtype)
            redraw.sort(axis=1)
            cols[bad] = redraw
        indices = cols.reshape(-1)
    else:
        lengths = np.full(n, per_row, dtype=np.int64)
        _, c = _distinct_sorted_columns(lengths, n, rng)
        indices = c.astype(index_dtype)
    data = rng.standard_normal(n * per_row, dtype=np.float32)
    indptr = (np.arange(n + 1, dtype=np.int64) * per_row).astype(index_dtype)
    return Matrix(f"random{per_row}_{n}", data, indices, indptr, (n, n))


def power_law(n: int = 2_097_152, alpha: float = 2.0, max_len: int = 200_000, seed: int = 0,
              index_dtype=np.int64) -> Matrix:
    rng = np.random.default_rng(seed)
    lengths = np.clip(rng.zipf(alpha, size=n), 1, min(max_len, n)).astype(np.int64)
    rows, cols = _distinct_sorted_columns(lengths, n, rng)
    data = (1.0 / lengths[rows]).astype(np.float32)
    return Matrix(f"powerlaw{alpha}_{n}", data, cols.astype(index_dtype),
                  _indptr_from_lengths(lengths, index_dtype), (n, n))


def banded(n: int = 1_048_576, half_band: int = 32, fill: float = 0.65, shift: float = 70.0,
           seed: int = 0, index_dtype=np.int32) -> Matrix:
    rng = np.random.default_rng(seed)
    offs = np.arange(-half_band, half_band + 1, dtype=np.int64)
    keep = rng.random((n, offs.size)) < fill
    keep[:, half_band] = True
    cols = np.arange(n, dtype=np.int64)[:, None] + offs[None, :]
    keep &= (cols >= 0) & (cols < n)
    lengths = keep.sum(axis=1)
    vals = rng.standard_normal((n, offs.size), dtype=np.float32)
    vals[:, half_band] += np.float32(shift)
    data = np.ascontiguousarray(vals[keep])
    return Matrix(f"banded{half_band}_{n}", data, cols[keep].astype(index_dtype),
                  _indptr_from_lengths(lengths, index_dtype), (n, n))


def uniform(n: int, low: float, high: float, seed: int, k: int | None = None) -> np.ndarray:
    rng = np.random.default_rng(seed)
    size = n if k is None else (n, k)
    return rng.uniform(low, high, size=size).astype(np.float32)


def normal(n: int, seed: int, k: int | None = None) -> np.ndarray:
    rng = np.random.default_rng(seed)
    size = n if k is None else (n, k)
    return rng.standard_normal(size, dtype=np.float32)


def complex_values(m: Matrix, seed: int) -> np.ndarray:
    """complex64 values with real and imaginary parts ~ N(0, 1)."""
    rng = np.random.default_rng(seed)
    re = rng.standard_normal(m.nnz, dtype=np.float32)
    im = rng.standard_normal(m.nnz, dtype=np.float32)
    return (re + 1j * im).astype(np.complex64)


def compulsory_bytes(nnz: int, n_rows: int, n_cols: int, value_bytes: int, index_bytes: int,
                     k: int = 1) -> int:
    """nnz*(value+index) + indptr + x (or X) once + y (or Y) once."""
    return (nnz * (value_bytes + index_bytes) + (n_rows + 1) * index_bytes
            + n_cols * value_bytes * k + n_rows * value_bytes * k)


def flops(nnz: int, k: int = 1, complex_values: bool = False) -> int:
    return (8 if complex_values else 2) * nnz * k
