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

The column-panel layout of a bound plan (csr_panel_build.hip; exported by
``msx_csr_plan_export_panels``) is restated by ``panel_layout``:

- x is cut into panels of PW = 131072 / acc_bytes columns (acc_bytes = 4 for
  float32/float16/bfloat16, 8 for complex64); tiles hold at most
  TW = 65536 / acc_bytes LDS words; H = TW - W;
- a short row (len(r) <= W) starts a tile when r == 0, row r-1 is long, or
  floor((s(r) + r) / H) != floor((s(r-1) + r-1) / H), s(r) = indptr[r]
  clamped to [0, nnz]; a tile runs to the next tile start or long row;
- every value p of a short row with a column c in [0, n_cols) and an LDS word
  (p - s(first row of its tile)) + (r - first row) below TW gets the segment
  key floor(c / PW) * n_tiles + tile; segment k holds the values with key k
  padded to a multiple of 4 entries, so ``seg_begin[k]`` is the sum over
  keys k' < k of ceil(count(k') / 4) * 4 (k = 0 .. n_panels * n_tiles).

Pinned by ``panel_layout_loop`` (plain per-row loops) and by the tile and
segment invariants in the same test file.
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


def panel_constants(acc_bytes: int, W: int):
    """(PW, TW, H) of a panel plan."""
    PW, TW = 131072 // acc_bytes, 65536 // acc_bytes
    return PW, TW, TW - W


def panel_layout(indptr, indices, n_cols: int, acc_bytes: int = 4, W: int = 256):
    """Returns (tile_begin, tile_end, seg_begin) as int64 arrays."""
    PW, TW, H = panel_constants(acc_bytes, W)
    p = np.asarray(indptr, dtype=np.int64)
    idx = np.asarray(indices, dtype=np.int64)
    n, nnz = len(p) - 1, len(idx)
    if n == 0:
        return np.zeros(0, np.int64), np.zeros(0, np.int64), np.zeros(1, np.int64)
    rows = np.arange(n, dtype=np.int64)
    long_ = (p[1:] - p[:-1]) > W
    s = np.clip(p[:-1], 0, nnz)
    e = np.maximum(np.clip(p[1:], 0, nnz), s)
    key = (s + rows) // H
    start = ~long_.copy()
    start[1:] &= long_[:-1] | (key[1:] != key[:-1])
    tile_begin = rows[start]
    nxt_break = np.ones(n, bool)
    nxt_break[:-1] = long_[1:] | start[1:]
    tile_end = rows[~long_ & nxt_break] + 1
    n_tiles = len(tile_begin)
    P = -(-n_cols // PW) if n_cols > 0 else 0
    tile_of = np.cumsum(start) - 1
    short_rows = rows[~long_]
    lens = (e - s)[~long_]
    pos = np.concatenate([np.arange(a, b) for a, b in zip(s[~long_], e[~long_])]) \
        if len(short_rows) else np.zeros(0, np.int64)
    r_of = np.repeat(short_rows, lens)
    T = tile_of[r_of]
    first = tile_begin[T]
    dest = (pos - s[first]) + (r_of - first)
    c = idx[pos] if len(pos) else np.zeros(0, np.int64)
    ok = (c >= 0) & (c < n_cols) & (dest >= 0) & (dest < TW)
    counts = np.bincount((c[ok] // PW) * n_tiles + T[ok], minlength=P * n_tiles)
    seg = np.concatenate([[0], np.cumsum((counts + 3) // 4 * 4)]).astype(np.int64)
    return tile_begin.astype(np.int64), tile_end.astype(np.int64), seg


def panel_layout_loop(indptr, indices, n_cols: int, acc_bytes: int = 4, W: int = 256):
    """Same layout with plain per-row loops (small inputs only)."""
    PW, TW, H = panel_constants(acc_bytes, W)
    p = [int(v) for v in indptr]
    idx = [int(v) for v in indices]
    n, nnz = len(p) - 1, len(idx)

    def clamp(v):
        return min(max(v, 0), nnz)

    tiles = []  # [first, last + 1]
    prev_long, prev_key = True, None
    for r in range(n):
        is_long = p[r + 1] - p[r] > W
        key = (clamp(p[r]) + r) // H
        if is_long:
            prev_long = True
            continue
        if prev_long or key != prev_key:
            tiles.append([r, r + 1])
        else:
            tiles[-1][1] = r + 1
        prev_long, prev_key = False, key
    n_tiles = len(tiles)
    P = -(-n_cols // PW) if n_cols > 0 else 0
    counts = [0] * (P * n_tiles)
    for t, (r0, r1) in enumerate(tiles):
        b0 = clamp(p[r0])
        for r in range(r0, r1):
            s = clamp(p[r])
            e = max(clamp(p[r + 1]), s)
            for q in range(s, e):
                c, dest = idx[q], (q - b0) + (r - r0)
                if 0 <= c < n_cols and 0 <= dest < TW:
                    counts[(c // PW) * n_tiles + t] += 1
    seg = [0]
    for v in counts:
        seg.append(seg[-1] + 4 * ((v + 3) // 4))
    return (np.array([a for a, _ in tiles], np.int64), np.array([b for _, b in tiles], np.int64),
            np.array(seg, np.int64))
