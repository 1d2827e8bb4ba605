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
