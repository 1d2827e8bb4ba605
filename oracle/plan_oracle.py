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
- virtual rows: a short row (len(r) <= W) is one, spanning [s(r), e(r)),
  s(r) = indptr[r] clamped to [0, nnz], e(r) = max(clamped indptr[r+1],
  s(r)); a long row is max(1, ceil((e(r) - s(r)) / C)) of them,
  C = min(W, 64), chunk k starting at min(s(r) + k C, nnz).  Virtual row v spans [vs(v), ve(v)),
  ve(v) = max(vs(v+1), vs(v)) with vs(n_v) = s(n);
- virtual row v starts a tile when v == 0 or
  floor((vs(v) + v) / H) != floor((vs(v-1) + v-1) / H); a tile runs to the
  next tile start (tile bounds are virtual-row numbers);
- every value p of virtual row v with a column c in [0, n_cols) and an LDS
  word (p - vs(first of its tile)) + (v - first) below TW gets the segment
  key floor(c / PW) * n_tiles + tile; segment k holds the values with key k
  padded to a multiple of 4 entries, so ``seg_begin[k]`` is the sum over
  keys k' < k of ceil(count(k') / 4) * 4 (k = 0 .. n_panels * n_tiles).

Without long rows the virtual rows are the rows.  ``virtual_slots`` gives
each virtual row's output slot (its row, or -1 - row for a chunk of a long
row) and each row's first virtual row.

Pinned by ``panel_layout_loop`` (plain per-row loops) and by the tile and
segment invariants in the same test file.
"""

from __future__ import annotations

import numpy as np


LONG_FLAG = 1 << 31
LONG_CHUNK = 64  # values per virtual row of a long row in the panel layout


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


def virtual_rows(indptr, nnz: int, W: int = 256):
    """(vs, ve, row) of the virtual rows: starts, ends and owning row."""
    p = np.asarray(indptr, dtype=np.int64)
    n = len(p) - 1
    s = np.clip(p[:-1], 0, nnz)
    e = np.maximum(np.clip(p[1:], 0, nnz), s)
    long_ = (p[1:] - p[:-1]) > W
    C = min(W, LONG_CHUNK)
    count = np.where(long_, np.maximum(1, -(-(e - s) // C)), 1)
    vbase = np.concatenate([[0], np.cumsum(count)]).astype(np.int64)
    nv = int(vbase[-1])
    row = np.repeat(np.arange(n, dtype=np.int64), count)
    k = np.arange(nv, dtype=np.int64) - vbase[row]
    vs = np.minimum(s[row] + k * C, nnz)
    vs_full = np.concatenate([vs, [np.clip(p[n], 0, nnz)]]) if n > 0 else np.zeros(1, np.int64)
    ve = np.maximum(vs_full[1:], vs)
    return vs.astype(np.int64), ve.astype(np.int64), row


def virtual_slots(indptr, nnz: int, W: int = 256):
    """(vslot, vbase) of the virtual rows (csr_panel_build.hip vrow_fill):
    vslot[v] = r for the one virtual row of a short row r, -1 - r for each
    chunk of a long row r; vbase[r] = the first virtual row of row r
    (vbase[n] = the number of virtual rows).  Pass 2 of the SpMV stores a
    virtual row's sum at y[vslot[v]] when vslot[v] >= 0, else at
    partial[v]; the long-row fixup adds partial[vbase[r] .. vbase[r+1]) into
    y[r]."""
    p = np.asarray(indptr, dtype=np.int64)
    n = len(p) - 1
    _, _, row = virtual_rows(p, nnz, W)
    long_ = (p[1:] - p[:-1]) > W
    vslot = np.where(long_[row], -1 - row, row).astype(np.int64)
    count = np.bincount(row, minlength=n) if n > 0 else np.zeros(0, np.int64)
    vbase = np.concatenate([[0], np.cumsum(count)]).astype(np.int64)
    return vslot, vbase


def virtual_slots_loop(indptr, nnz: int, W: int = 256):
    """Same as ``virtual_slots`` with a plain per-row loop."""
    p = [int(v) for v in indptr]
    n = len(p) - 1
    C = min(W, LONG_CHUNK)
    vslot, vbase = [], [0]
    for r in range(n):
        s = min(max(p[r], 0), nnz)
        e = max(min(max(p[r + 1], 0), nnz), s)
        if p[r + 1] - p[r] > W:
            for _ in range(max(1, (e - s + C - 1) // C)):
                vslot.append(-1 - r)
        else:
            vslot.append(r)
        vbase.append(len(vslot))
    return np.array(vslot, np.int64), np.array(vbase, np.int64)


def panel_layout(indptr, indices, n_cols: int, acc_bytes: int = 4, W: int = 256):
    """Returns (tile_begin, tile_end, seg_begin) as int64 arrays."""
    PW, TW, H = panel_constants(acc_bytes, W)
    p = np.asarray(indptr, dtype=np.int64)
    idx = np.asarray(indices, dtype=np.int64)
    n, nnz = len(p) - 1, len(idx)
    if n == 0:
        return np.zeros(0, np.int64), np.zeros(0, np.int64), np.zeros(1, np.int64)
    vs, ve, _ = virtual_rows(p, nnz, W)
    nv = len(vs)
    v = np.arange(nv, dtype=np.int64)
    key = (vs + v) // H
    start = np.ones(nv, bool)
    start[1:] = key[1:] != key[:-1]
    tile_begin = v[start]
    tile_end = np.concatenate([tile_begin[1:], [nv]])
    n_tiles = len(tile_begin)
    P = -(-n_cols // PW) if n_cols > 0 else 0
    tile_of = np.cumsum(start) - 1
    lens = ve - vs
    pos = np.concatenate([np.arange(a, b) for a, b in zip(vs, ve)]) if nv else np.zeros(0, np.int64)
    v_of = np.repeat(v, lens)
    T = tile_of[v_of]
    first = tile_begin[T]
    dest = (pos - vs[first]) + (v_of - first)
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

    starts = []  # virtual-row starts, then the end sentinel
    for r in range(n):
        s, e = clamp(p[r]), max(clamp(p[r + 1]), clamp(p[r]))
        if p[r + 1] - p[r] > W:
            C = min(W, LONG_CHUNK)
            for k in range(max(1, (e - s + C - 1) // C)):
                starts.append(min(s + k * C, nnz))
        else:
            starts.append(s)
    nv = len(starts)
    starts.append(clamp(p[n]) if n > 0 else 0)
    tiles = []  # [first, last + 1]
    prev_key = None
    for v in range(nv):
        key = (starts[v] + v) // H
        if v == 0 or key != prev_key:
            tiles.append([v, v + 1])
        else:
            tiles[-1][1] = v + 1
        prev_key = key
    n_tiles = len(tiles)
    P = -(-n_cols // PW) if n_cols > 0 else 0
    counts = [0] * (P * n_tiles)
    for t, (v0, v1) in enumerate(tiles):
        b0 = starts[v0]
        for v in range(v0, v1):
            s = starts[v]
            e = max(starts[v + 1], s)
            for q in range(s, e):
                c, dest = idx[q], (q - b0) + (v - v0)
                if 0 <= c < n_cols and 0 <= dest < TW:
                    counts[(c // PW) * n_tiles + t] += 1
    seg = [0]
    for v in counts:
        seg.append(seg[-1] + 4 * ((v + 3) // 4))
    return (np.array([a for a, _ in tiles], np.int64), np.array([b for _, b in tiles], np.int64),
            np.array(seg, np.int64))
