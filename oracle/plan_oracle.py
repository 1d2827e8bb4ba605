"""Row-block plan restated in numpy - TEST INFRASTRUCTURE ONLY.

The GPU plan (mlx-sparse_amd/csrc/csr_plan.hip) is this build's own index
structure, not a reference algorithm; the reference picks one kernel per
launch from ``nnz >= 32 * n_rows`` (reference:
src/sparse/csr_matvec/csr_matvec.cpp:291-296).  Its index work must match
this restatement bit for bit.  The rule, per row r with length
len(r) = indptr[r+1] - indptr[r]:

- r is long when len(r) > W; a long row has ceil(len / C) chunks;
- a row that is not long starts a short block when r == 0, r % R == 0,
  row r-1 is long, or floor(indptr[r] / W) != floor(indptr[r-1] / W);
- ``bounds`` lists, in row order, every block-start row and every long row,
  long rows with bit 31 set, then the sentinel n; a short block spans its
  entry up to the next entry.

Pinned in tests/test_plan_oracle.py by a per-row pure-Python loop and by the
block invariants (coverage, < 2W values, <= R rows).
"""

from __future__ import annotations

import numpy as np


LONG_FLAG = 1 << 31


def plan(indptr, W: int = 256, R: int = 256, C: int = 4096):
    """Returns (bounds incl. sentinel n, long_rows, long_chunk_begin incl.
    sentinel n_chunks) as int64 arrays."""
    p = np.asarray(indptr, dtype=np.int64)
    n = p.shape[0] - 1
    if n <= 0:
        return np.array([max(n, 0)], np.int64), np.zeros(0, np.int64), np.zeros(1, np.int64)
    length = p[1:] - p[:-1]
    is_long = length > W
    r = np.arange(n)
    start = np.zeros(n, bool)
    start[0] = True
    start[r % R == 0] = True
    window = np.floor_divide(p[:-1], W)
    start[1:] |= is_long[:-1] | (window[1:] != window[:-1])
    start &= ~is_long
    entries = np.nonzero(start | is_long)[0].astype(np.int64)
    entries = entries | np.where(is_long[entries], LONG_FLAG, 0)
    blocks = np.concatenate([entries, [n]]).astype(np.int64)
    long_rows = np.nonzero(is_long)[0].astype(np.int64)
    chunks = -(-length[long_rows] // C)
    chunk_begin = np.concatenate([[0], np.cumsum(chunks)]).astype(np.int64)
    return blocks, long_rows, chunk_begin


def plan_loop(indptr, W: int = 256, R: int = 256, C: int = 4096):
    """Same rule as ``plan`` with plain per-row loops (small inputs only)."""
    p = [int(v) for v in indptr]
    n = len(p) - 1
    blocks, longs, chunk_begin = [], [], [0]
    for r in range(n):
        ln = p[r + 1] - p[r]
        if ln > W:
            longs.append(r)
            blocks.append(r + LONG_FLAG)
            chunk_begin.append(chunk_begin[-1] + (ln + C - 1) // C)
            continue
        prev_long = r > 0 and p[r] - p[r - 1] > W
        if r == 0 or r % R == 0 or prev_long or p[r] // W != p[r - 1] // W:
            blocks.append(r)
    blocks.append(max(n, 0))
    return (np.array(blocks, np.int64), np.array(longs, np.int64), np.array(chunk_begin, np.int64))
