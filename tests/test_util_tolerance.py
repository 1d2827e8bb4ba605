"""The per-row parity helper itself: a result outside the bound fails, and so
does any non-finite result that the oracle does not share (NaN - x is NaN,
and a comparison with NaN is False, so ``err > bound`` alone would let it
pass)."""

from __future__ import annotations

import numpy as np
import pytest

from _util import assert_rows_close, storage

SCALE = np.array([1.0, 1.0])


def _check(got, want, vtype="float32", scale=SCALE):
    return assert_rows_close(storage(np.array(got), vtype), storage(np.array(want), vtype),
                             np.asarray(scale, np.float64), vtype, "helper")


@pytest.mark.parametrize("vtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf])
def test_nonfinite_against_finite_fails(vtype, bad):
    with pytest.raises(AssertionError):
        _check([bad, 1.0], [1.0, 1.0], vtype)
    with pytest.raises(AssertionError):
        _check([1.0, 1.0], [1.0, bad], vtype)


@pytest.mark.parametrize("vtype", ["float32", "float16", "bfloat16"])
def test_same_nonfinite_passes(vtype):
    assert _check([np.nan, np.inf], [np.nan, np.inf], vtype)["rows_outside_tol_vs_oracle"] == 0
    assert _check([-np.inf, 2.0], [-np.inf, 2.0], vtype)["rows_outside_tol_vs_oracle"] == 0


def test_opposite_infinities_fail():
    with pytest.raises(AssertionError):
        _check([np.inf, 1.0], [-np.inf, 1.0])


def test_nan_against_inf_fails():
    with pytest.raises(AssertionError):
        _check([np.nan, 1.0], [np.inf, 1.0])


def test_nan_scale_fails():
    # a bound that is NaN (non-finite scale) admits nothing
    with pytest.raises(AssertionError):
        _check([1.0, 1.0], [1.0, 1.0], scale=[np.nan, 1.0])


def test_bound_edges():
    assert _check([1.0 + 1e-6, 1.0], [1.0, 1.0])["rows_outside_tol_vs_oracle"] == 0
    with pytest.raises(AssertionError):
        _check([1.0 + 1e-4, 1.0], [1.0, 1.0])


@pytest.mark.parametrize("bad", [complex(np.nan, 0.0), complex(0.0, np.nan), complex(np.inf, 1.0),
                                 complex(1.0, -np.inf)])
def test_complex_nonfinite_component_fails(bad):
    with pytest.raises(AssertionError):
        _check([bad, 1.0], [1.0 + 1.0j, 1.0], "complex64")


def test_complex_same_nonfinite_passes():
    got = [complex(np.inf, 2.0), complex(np.nan, np.nan)]
    assert _check(got, got, "complex64")["rows_outside_tol_vs_oracle"] == 0
    with pytest.raises(AssertionError):  # same infinite real part, other imaginary part
        _check([complex(np.inf, 2.0), 0], [complex(np.inf, 3.0), 0], "complex64")


def test_exempt_rows_never_admit_nan():
    exact = np.array([1.0, 1.0])
    with pytest.raises(AssertionError):
        assert_rows_close(storage(np.array([np.nan, 1.0]), "float32"),
                          storage(np.array([1.5, 1.0]), "float32"), SCALE, "float32", "exempt",
                          exact=exact, lengths=np.array([20000, 1]), min_len_exempt=10)
