"""The parity helpers' handling of infinities and NaN (CPU only)."""
import numpy as np

from tests.netgen import close, max_rel

INF, NAN = np.inf, np.nan


def test_equal_values_agree_even_when_not_finite():
    # a diverging network compares by where it overflowed: matching infinities
    # and matching NaN count as agreement
    assert max_rel([1.0, INF, -INF, NAN], [1.0, INF, -INF, NAN]) == 0.0
    assert close([2.0, INF], [2.0, INF], 1e-4)


def test_one_sided_non_finite_values_fail():
    for a, b in (([INF], [1.0]), ([1.0], [INF]), ([NAN], [1.0]), ([1.0], [NAN]), ([INF], [-INF]), ([NAN], [INF])):
        assert max_rel(a, b) == INF, (a, b)
        assert not close(a, b, 1e-4), (a, b)


def test_no_nan_reaches_a_reduction():
    # Python's max() keeps its first argument when a later one is NaN; the
    # helper never returns NaN, so a per-layer max over it sees every layer
    layers = [([1.0], [1.0]), ([NAN], [2.0]), ([3.0], [3.0])]
    assert max(max_rel(a, b) for a, b in layers) == INF


def test_finite_bound_is_the_reference_tests():
    # |a-b| / (1+|b|), BatchedPcForwardTests.cs:67
    assert abs(max_rel([1.5], [1.0]) - 0.25) < 1e-12
    assert close([1.0 + 1e-4], [1.0], 1e-4) and not close([1.0 + 3e-4], [1.0], 1e-4)
    assert max_rel([], []) == 0.0
