"""Pins the numpy restatement of the row-block plan (oracle/plan_oracle.py)
against a per-row loop and against the invariants the kernels rely on."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import plan_oracle


def _indptr(rng, n, kind):
    if kind == "uniform":
        lengths = np.full(n, 16)
    elif kind == "mixed":
        lengths = rng.integers(0, 40, n)
        big = rng.random(n) < 0.05
        lengths[big] = rng.integers(257, 9000, big.sum())
    elif kind == "empty":
        lengths = np.zeros(n, np.int64)
        lengths[::97] = 3
    else:  # power law
        lengths = np.clip(rng.zipf(1.8, n), 1, 20000)
    p = np.zeros(n + 1, np.int64)
    np.cumsum(lengths, out=p[1:])
    return p


@pytest.mark.parametrize("kind", ["uniform", "mixed", "empty", "zipf"])
@pytest.mark.parametrize("W", [64, 256, 512, 1024])
def test_vectorised_rule_matches_loop(kind, W):
    rng = np.random.default_rng(W)
    p = _indptr(rng, 3000, kind)
    a = plan_oracle.plan(p, W=W)
    b = plan_oracle.plan_loop(p, W=W)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)


@pytest.mark.parametrize("kind", ["uniform", "mixed", "empty", "zipf"])
def test_block_invariants(kind):
    W, R, C = 512, 256, 4096
    rng = np.random.default_rng(3)
    p = _indptr(rng, 5000, kind)
    bounds, longs, chunk_begin = plan_oracle.plan(p, W=W, R=R, C=C)
    lengths = np.diff(p)
    flag = plan_oracle.LONG_FLAG
    rows = bounds & (flag - 1)
    assert np.all(np.diff(rows) > 0)  # strictly increasing entries
    covered = np.zeros(len(lengths), int)
    for e, nxt in zip(bounds[:-1], rows[1:]):
        r0 = e & (flag - 1)
        if e & flag:
            assert lengths[r0] > W
            covered[r0] += 1
            continue
        block = np.arange(r0, nxt)
        assert np.all(lengths[block] <= W)  # never contains a long row
        assert len(block) <= R
        assert p[block[-1] + 1] - p[block[0]] < 2 * W
        covered[block] += 1
    assert np.all(covered == 1)
    np.testing.assert_array_equal(rows[:-1][bounds[:-1] >= flag], longs)
    np.testing.assert_array_equal(np.diff(chunk_begin), -(-lengths[longs] // C))


def test_empty_matrix():
    blocks, longs, cb = plan_oracle.plan(np.zeros(1, np.int64))
    assert blocks.tolist() == [0] and longs.size == 0 and cb.tolist() == [0]


# -- column-panel layout ------------------------------------------------------------

def _panel_case(rng, kind, n=3000, n_cols=70000):
    p = _indptr(rng, n, kind)
    idx = rng.integers(0, n_cols, int(p[-1]))
    if kind == "mixed":  # a few malformed columns, dropped from the copy
        bad = rng.random(len(idx)) < 0.01
        idx[bad] = np.where(rng.random(int(bad.sum())) < 0.5, -1, n_cols + 5)
    return p, idx, n_cols


@pytest.mark.parametrize("kind", ["uniform", "mixed", "empty", "zipf"])
@pytest.mark.parametrize("acc_bytes,W", [(4, 256), (4, 64), (8, 1024)])
def test_panel_layout_matches_loop(kind, acc_bytes, W):
    rng = np.random.default_rng(acc_bytes * W)
    p, idx, n_cols = _panel_case(rng, kind)
    a = plan_oracle.panel_layout(p, idx, n_cols, acc_bytes, W)
    b = plan_oracle.panel_layout_loop(p, idx, n_cols, acc_bytes, W)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)


@pytest.mark.parametrize("kind", ["uniform", "mixed", "empty", "zipf"])
@pytest.mark.parametrize("acc_bytes", [4, 8])
def test_panel_layout_invariants(kind, acc_bytes):
    W = 256
    rng = np.random.default_rng(11)
    p, idx, n_cols = _panel_case(rng, kind, n=20000, n_cols=200000)
    PW, TW, H = plan_oracle.panel_constants(acc_bytes, W)
    tb, te, seg = plan_oracle.panel_layout(p, idx, n_cols, acc_bytes, W)
    lengths = np.diff(p)
    vs, ve, row = plan_oracle.virtual_rows(p, int(p[-1]), W)
    nv = len(vs)
    # virtual rows: at most W values each; a row's virtual rows are
    # consecutive, cover its values in order, and only long rows have more
    # than one
    assert np.all(ve - vs <= W) and np.all(ve >= vs)
    np.testing.assert_array_equal(np.bincount(row, ve - vs, minlength=len(lengths)), lengths)
    per_row = np.bincount(row, minlength=len(lengths))
    assert np.all(per_row[lengths <= W] == 1)
    C = min(W, plan_oracle.LONG_CHUNK)
    np.testing.assert_array_equal(per_row[lengths > W], -(-lengths[lengths > W] // C))
    np.testing.assert_array_equal(vs[1:], ve[:-1])  # well-formed indptr: contiguous
    # tiles partition the virtual rows; products + one word per virtual row fit
    assert tb[0] == 0 and te[-1] == nv
    np.testing.assert_array_equal(tb[1:], te[:-1])
    for a, b in zip(tb, te):
        assert a < b
        assert (ve[b - 1] - vs[a]) + (b - a) <= TW
    # segments partition the valid values by (panel, tile), each padded to a
    # multiple of 4 entries
    n_tiles, P = len(tb), -(-n_cols // PW)
    assert len(seg) == P * n_tiles + 1 and seg[0] == 0 and np.all(np.diff(seg) >= 0)
    assert np.all(seg % 4 == 0)
    counts = np.zeros(P * n_tiles, np.int64)
    for t, (a, b) in enumerate(zip(tb, te)):
        cols = idx[vs[a]:ve[b - 1]]
        cols = cols[(cols >= 0) & (cols < n_cols)]
        np.add.at(counts, (cols // PW) * n_tiles + t, 1)
    np.testing.assert_array_equal(np.diff(seg), -(-counts // 4) * 4)
    assert np.all(np.diff(seg) - counts < 4)
    assert counts.sum() == int(((idx >= 0) & (idx < n_cols)).sum())


@pytest.mark.parametrize("kind", ["uniform", "mixed", "empty", "zipf"])
@pytest.mark.parametrize("W", [256, 512])
def test_virtual_slots_stay_in_bounds(kind, W):
    """Pass 2 of the panel SpMV (``panel_rows<..., true>``) runs over virtual
    rows, which outnumber the rows when rows are long; it may store only
    through ``vslot`` (y) or at the virtual row itself (partial).  Pinned
    against the per-row loop, then every store index is checked: a short
    virtual row's slot is a row in [0, n) and each such row is written once,
    a chunk's slot names a long row, its partial index lies in [0, n_v), and
    the fixup's ranges vbase[r] .. vbase[r+1] cover exactly the chunks of
    long row r.  Indexing y by the virtual row instead would write past y
    whenever n_v > n."""
    rng = np.random.default_rng(7 + W)
    p = _indptr(rng, 4000, kind)
    nnz = int(p[-1])
    vslot, vbase = plan_oracle.virtual_slots(p, nnz, W=W)
    ls, lb = plan_oracle.virtual_slots_loop(p, nnz, W=W)
    np.testing.assert_array_equal(vslot, ls)
    np.testing.assert_array_equal(vbase, lb)
    n = len(p) - 1
    nv = len(vslot)
    assert vbase[-1] == nv
    tb, te, _ = plan_oracle.panel_layout(p, np.zeros(nnz, np.int64), 1, W=W)
    assert tb[0] == 0 and te[-1] == nv and np.all(tb < te) and np.all(tb[1:] == te[:-1])
    long_ = (p[1:] - p[:-1]) > W
    short_v = vslot >= 0
    # y stores: rows in [0, n), every short row exactly once, no long row
    assert np.all(vslot[short_v] < n)
    np.testing.assert_array_equal(np.bincount(vslot[short_v], minlength=n), (~long_).astype(np.int64))
    # partial stores: chunks of long rows, indexed by the virtual row < n_v
    chunk_rows = -1 - vslot[~short_v]
    assert np.all((chunk_rows >= 0) & (chunk_rows < n)) and np.all(long_[chunk_rows])
    for r in np.flatnonzero(long_):
        assert np.all(vslot[vbase[r]:vbase[r + 1]] == -1 - r)
        assert vbase[r + 1] > vbase[r]
    if kind in ("mixed", "zipf"):
        assert nv > n  # y[v] for every virtual row v would run past y
