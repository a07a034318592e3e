"""The timing protocol's statistics and visiting order (CPU; no events are recorded)."""
from __future__ import annotations

from techjam2026_amd.timing import Timing, visit_order


def test_statistics_closed_forms():
    t = Timing([4.0, 1.0, 3.0, 2.0, 5.0], [0, 0, 1, 1, 2])
    assert t.median_ms == 3.0
    assert t.min_ms == 1.0
    assert t.mean_ms == 3.0
    # linear interpolation between the 4th and 5th order statistics: 4 + 0.6 * 1
    assert abs(t.p90_ms - 4.6) < 1e-12
    assert abs(t.spread - 4.6) < 1e-12
    assert t.round_medians() == [2.5, 2.5, 5.0]


def test_even_count_median_and_steady_spread():
    assert Timing([1.0, 2.0]).median_ms == 1.5
    assert Timing([2.0] * 7).spread == 1.0


def test_rounds_rotate_so_no_candidate_is_always_last():
    order = visit_order(["ref", "a", "b"], 3)
    assert order == [["ref", "a", "b"], ["a", "b", "ref"], ["b", "ref", "a"]]
    assert {o[-1] for o in order} == {"ref", "a", "b"}
    assert visit_order([], 2) == [[], []]
