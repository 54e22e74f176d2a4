"""The comparison helpers of tests/_helpers.py: relative bars with the
small-element floor, and the summation-order variant's outlier budget."""
import numpy as np
import pytest

from _helpers import assert_close_rel, assert_close_rel_summation


def test_relative_bar_and_floor():
    e = np.array([100.0, 1.0, 1e-6])
    assert_close_rel(e * (1 + 9e-4), e, 1e-3)
    with pytest.raises(AssertionError):
        assert_close_rel(e * (1 + 2e-3), e, 1e-3)
    # elements below 1e-2 of the largest magnitude are held to rtol * (1e-2 * 100)
    assert assert_close_rel(e + np.array([0.0, 0.0, 5e-4]), e, 1e-3) == 1
    # the ordered-results floor, 1e-4 of the largest, holds them to 1e-5 absolute
    with pytest.raises(AssertionError):
        assert_close_rel(e + np.array([0.0, 0.0, 5e-4]), e, 1e-3, floor_rel=1e-4)
    assert assert_close_rel(e + np.array([0.0, 0.0, 5e-6]), e, 1e-3, floor_rel=1e-4) == 1
    assert assert_close_rel(e * (1 + 9e-4), e, 1e-3, floor_rel=1e-4) == 0


def test_summation_outlier_budget():
    rng = np.random.default_rng(0)
    e = rng.uniform(1.0, 2.0, 3_000_000)
    a = e.copy()
    a[[5, 77]] *= 1 + 5e-3  # two elements past 1e-3, within 1e-2: allowed (budget max(2, 3))
    assert_close_rel_summation(a, e, 1e-3)
    a[1000:1010] *= 1 + 5e-3  # twelve: over the budget
    with pytest.raises(AssertionError, match="beyond"):
        assert_close_rel_summation(a, e, 1e-3)
    b = e.copy()
    b[3] *= 1 + 5e-2  # one element past 1e-2: never allowed
    with pytest.raises(AssertionError):
        assert_close_rel_summation(b, e, 1e-3)
