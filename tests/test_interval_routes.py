"""Interval routes of equality-or-range query sets (plan.interval_route_rows).

Pinned against a brute-force overlap test over the integer intervals, against
the pure-range cover planner (plan_pure_range_cover, the restatement of
dataloader.cpp:9204-9345) over a one-level layout of the same intervals, and
against the interval every row of the synthetic generator is labelled with.
"""
from __future__ import annotations

import numpy as np
import pytest

from gofann_amd import plan as gp

U = 0xFFFFFFFF


class _Index:
    def __init__(self, graphs):
        self.graphs = set(graphs)

    def has_graph(self, label):
        return label in self.graphs


def _bounds(intervals, attr_max):
    # interval i holds the integers v with floor(v * intervals / attr_max) == i
    v = np.arange(attr_max)
    iv = v * intervals // attr_max
    return [(int(v[iv == i].min()), int(v[iv == i].max()) + 1) for i in range(intervals)]


def _layout(cats, intervals, attr_max):
    b = _bounds(intervals, attr_max)
    n = cats + intervals
    iv = gp.RangeLabelIntervals(1, np.zeros(n, np.uint8), np.zeros(n, np.float32),
                                np.zeros(n, np.float32), np.full(n, U, np.uint32),
                                np.full(n, U, np.uint32), np.zeros(n, np.uint32))
    for i, (lo, hi) in enumerate(b):
        lab = cats + i
        iv.has_interval[lab] = 1
        iv.lower[lab], iv.upper[lab] = lo, hi
        iv.level[lab], iv.bin[lab] = 0, i
    return gp.build_range_cover_layout(iv, 0)


@pytest.mark.parametrize("intervals,attr_max", [(10, 1000), (7, 1000), (100, 12345), (3, 5)])
def test_range_routes_are_the_overlapping_intervals(intervals, attr_max):
    cats = 4
    rng = np.random.default_rng(intervals * 7 + attr_max)
    bounds = _bounds(intervals, attr_max)
    layout = _layout(cats, intervals, attr_max)
    qlabels, qranges = [], []
    for _ in range(300):
        lo = int(rng.integers(0, attr_max))
        hi = int(rng.integers(lo + 1, attr_max + 1))
        qlabels.append([])
        qranges.append([(0, 3, float(lo), float(hi))])
    g, p, interior = gp.interval_route_rows(_Index([]), qlabels, qranges, cats, intervals,
                                            attr_max)
    assert p == []
    by_q = {}
    for q, lab, rl, rr in g:
        by_q.setdefault(q, []).append((lab, rl, rr))
    n_inside = 0
    for q, ((_, _, lo, hi),) in enumerate(qranges):
        lo, hi = int(lo), int(hi)
        want = [i for i, (a, b) in enumerate(bounds) if a < hi and b > lo]  # brute force
        got = by_q[q]
        assert [lab - cats for lab, _, _ in got] == want
        assert [lab for lab, _, _ in got] == gp.plan_pure_range_cover(
            layout, 3, lo, hi, finest_only=True)
        for lab, rl, rr in got:
            a, b = bounds[lab - cats]
            inside = lo <= a and b <= hi
            n_inside += inside
            assert rl == []
            # the range is a residual exactly where the interval is not
            # wholly inside it
            assert rr == ([] if inside else [(0, 3, float(lo), float(hi))])
    assert interior == n_inside


def test_equality_routes_take_a_graph_or_a_posting():
    cats, intervals, attr_max = 6, 10, 100
    qlabels = [[0], [1], [], [5], [2]]
    qranges = [[], [], [(0, 3, 15.0, 35.0)], [], []]
    g, p, interior = gp.interval_route_rows(_Index([0, 2, 5]), qlabels, qranges, cats,
                                            intervals, attr_max)
    assert p == [(1, 1, [], [])]
    assert g == [(0, 0, [], []),
                 (2, cats + 1, [], [(0, 3, 15.0, 35.0)]),
                 (2, cats + 2, [], []),
                 (2, cats + 3, [], [(0, 3, 15.0, 35.0)]),
                 (3, 5, [], []),
                 (4, 2, [], [])]
    assert interior == 1


def test_generator_rows_sit_in_the_routes_of_the_ranges_holding_them():
    # every row whose attribute lies in a query's range carries an interval
    # label among that query's routes (the routes cover the range)
    from gofann_amd import synth
    wl = synth.config4(n=3000, nq=40, device="cpu", dim=8, k=4, rank=2)
    cats, nint, amax = wl.meta["categories"], wl.meta["intervals"], wl.meta["attr_max"]
    g, _, _ = gp.interval_route_rows(_Index([]), wl.query_labels, wl.query_ranges, cats, nint,
                                     amax)
    routes = {}
    for q, lab, _, _ in g:
        routes.setdefault(q, set()).add(lab)
    attr = wl.base_ranges[:, 0].astype(np.int64)
    row_interval = wl.label_values[1::2]
    checked = 0
    for q, rr in enumerate(wl.query_ranges):
        if not rr:
            continue
        (_, _, lo, hi), = rr
        hit = (attr >= lo) & (attr < hi)
        assert set(row_interval[hit].tolist()) <= routes[q]
        checked += int(hit.sum())
    assert checked > 0


def test_only_one_half_open_range_on_dimension_0():
    with pytest.raises(ValueError):
        gp.interval_route_rows(_Index([]), [[]], [[(0, 1, 5.0, 0.0)]], 2, 10, 100)
