"""The bench's recall figure and its beam rule, on hand-computed cases.

`bench.recall_at_10` is the macro recall of the reference's evaluator
(scripts/evaluate.py:163-203): per query, the distinct predicted ids among
the first 10 that are in its ground truth, over the ground-truth size;
padding ids (UINT32_MAX, i.e. -1) never count; queries whose ground truth is
empty are left out of the mean.  `bench.reaches` accepts a beam when the
mean minus 1.96 standard errors of the per-query recalls clears the target.
"""
from __future__ import annotations

import math

import numpy as np

import bench

PAD = np.uint32(0xFFFFFFFF)


def _rows(*rows):
    out = np.full((len(rows), 10), PAD, dtype=np.uint32)
    for i, r in enumerate(rows):
        out[i, :len(r)] = r
    return out


def test_macro_recall_known_answers():
    res = _rows([1, 2, 9, 8], [5, 5, 5], [7], [3, 4])
    gt = {0: np.array([1, 2, 3, 4], np.uint32),   # 2 of 4
          1: np.array([5], np.uint32),            # 1 of 1, the repeats count once
          3: np.array([4, 3, 6], np.uint32)}      # 2 of 3; query 2 has no ground truth
    assert math.isclose(bench.recall_at_10(res, gt), (0.5 + 1.0 + 2 / 3) / 3)


def test_padding_and_empty_ground_truth_do_not_count():
    res = _rows([], [1])
    # an all-padding row scores 0 against a real ground truth; a query with an
    # empty ground truth is left out, not counted as 0 or 1
    gt = {0: np.array([1, 2], np.uint32), 1: np.array([], np.uint32)}
    assert bench.recall_at_10(res, gt) == 0.0
    gt = {1: np.array([1], np.uint32), 0: np.array([], np.uint32)}
    assert bench.recall_at_10(res, gt) == 1.0


def test_only_the_first_ten_predictions_count():
    res = _rows(list(range(10)))
    gt = {0: np.array([3, 10, 11], np.uint32)}  # 10 and 11 would be ranks 11 and 12
    assert math.isclose(bench.recall_at_10(res, gt), 1 / 3)


def test_reaches_uses_the_lower_95_percent_bound():
    # 100 queries: 90 at recall 1, 10 at recall 0 -> mean 0.9, sample standard
    # deviation sqrt(100/99 * 0.09), standard error that / 10
    res = _rows(*([[1]] * 100))
    gt = {q: np.array([1 if q < 90 else 2], np.uint32) for q in range(100)}
    assert math.isclose(bench.recall_at_10(res, gt), 0.9)
    lower = 0.9 - 1.96 * math.sqrt(100 / 99 * 0.09) / 10
    assert bench.reaches(res, gt, lower - 1e-9)
    assert not bench.reaches(res, gt, lower + 1e-9)
    # the mean alone would pass 0.9; the bound does not
    assert not bench.reaches(res, gt, 0.9)


def test_reaches_with_no_ground_truth_is_vacuous():
    res = _rows([1])
    assert bench.reaches(res, {}, 0.9)
    assert bench.reaches(res, {0: np.array([1], np.uint32)}, 1.0)
