"""Pure-range cover planner (plan_pure_range_cover_labels, dataloader.cpp:
9104-9345) and the range label manifest (load_range_label_manifest,
:6883-7001), CPU only: the reference's own coarsening fixture, and random
hierarchies against an independent statement of the canonical cover."""
from __future__ import annotations

import json

import numpy as np
import pytest

from gofann_amd import plan as gp

U32MAX = 0xFFFFFFFF


def test_coarsening_reference_fixture():
    # tests/native/graph_route_selection_test.cpp:117-135
    children = np.zeros(32, np.uint8)
    children[8:16] = 1
    children[16] = children[17] = 1
    parents = np.zeros(4, np.uint8)
    gp.coarsen_range_cover_bins(children, parents, np.array([100, 101, 102, 103], np.uint32))
    assert parents.tolist() == [0, 1, 0, 0]
    assert not children[8:16].any()
    assert children[16] == 1 and children[17] == 1


def test_coarsening_rejects_ragged_levels():
    with pytest.raises(ValueError, match="integer-multiple"):
        gp.coarsen_range_cover_bins(np.zeros(10, np.uint8), np.zeros(4, np.uint8),
                                    np.zeros(4, np.uint32))


def _hierarchy(bins, lo, hi, missing, rng):
    """Equal-width bins per level, labels numbered level by level; a random
    share of non-finest labels is left out of the manifest (never a level's
    last bin: the layout sizes a level by its highest bin, and the reference
    rejects levels whose bin counts are not integer multiples)."""
    levels, lab = [], 0
    for li, nb in enumerate(bins):
        edges = np.linspace(lo, hi, nb + 1).astype(np.float32)
        parts = []
        for b in range(nb):
            if li < len(bins) - 1 and b < nb - 1 and rng.random() < missing:
                lab += 1
                continue
            parts.append({"label_id": lab, "interval": [float(edges[b]), float(edges[b + 1])],
                          "bin_index": b})
            lab += 1
        levels.append({"level_index": li, "partitions": parts})
    return levels, lab


def _brute_cover(bins, levels, lo, hi, mode, qlo, qhi):
    """Independent statement: a finest bin is full when it overlaps the
    target; a coarser bin is full when it has a label and all its children
    are full; a full bin is chosen unless its parent is full."""
    f32 = np.float32
    tlo, thi = f32(lo), f32(hi)
    if mode in (1, 3):
        tlo = max(tlo, f32(qlo))
    if mode in (2, 3):
        thi = min(thi, f32(qhi))
    if mode == 0 or not tlo < thi:
        return []
    present = [{p["bin_index"]: p for p in lv["partitions"]} for lv in levels]
    top = len(bins) - 1
    eps = f32(1e-6)
    full = [None] * len(bins)
    full[top] = [b in present[top] and f32(present[top][b]["interval"][1]) > tlo + eps
                 and f32(present[top][b]["interval"][0]) < thi - eps for b in range(bins[top])]
    for li in range(top - 1, -1, -1):
        per = bins[li + 1] // bins[li]
        full[li] = [b in present[li] and all(full[li + 1][b * per:(b + 1) * per])
                    for b in range(bins[li])]
    chosen = []
    for li in range(len(bins)):
        for b in range(bins[li]):
            if not full[li][b]:
                continue
            if li > 0 and full[li - 1][b // (bins[li] // bins[li - 1])]:
                continue
            p = present[li][b]
            chosen.append((p["interval"][0], p["label_id"]))
    return [lab for _, lab in sorted(chosen)]


@pytest.mark.parametrize("bins", [[4, 16, 64], [3, 12, 48, 96], [1, 10], [5]])
@pytest.mark.parametrize("missing", [0.0, 0.3])
def test_cover_matches_brute_force(tmp_path, bins, missing):
    rng = np.random.default_rng(len(bins) * 100 + int(missing * 10))
    levels, nlab = _hierarchy(bins, 0.0, 1000.0, missing, rng)
    path = tmp_path / "manifest.json"
    path.write_text(json.dumps({"levels": levels}))
    iv = gp.load_range_label_manifest(str(path), nlab)
    layout = gp.build_range_cover_layout(iv, 0)
    edges = np.linspace(0, 1000, bins[-1] + 1)
    for _ in range(300):
        mode = int(rng.integers(0, 4))
        a, b = sorted(rng.uniform(-50, 1050, size=2))
        if rng.random() < 0.3:                       # land on bin edges
            a, b = sorted(rng.choice(edges, size=2, replace=False))
        want = _brute_cover(bins, levels, 0.0, 1000.0, mode, a, b)
        got = gp.plan_pure_range_cover(layout, mode, a, b)
        assert got == want, (mode, a, b)
        # every selected interval overlaps the target, and they tile it
        if got:
            fin = gp.plan_pure_range_cover(layout, mode, a, b, finest_only=True)
            assert len(fin) >= len(got)
            assert all(iv.level[l] == len(bins) - 1 for l in fin)


def test_manifest_ranges_layout(tmp_path):
    m = {"ranges": [
        {"range_index": 0, "levels": [{"level_index": 0, "partitions": [
            {"label_id": 2, "interval": [0, 10], "bin_index": 0},
            {"label_id": 3, "interval": [10, 20], "bin_index": 1}]}]},
        {"levels": [{"level_index": 0, "partitions": [
            {"label_id": 5, "interval": [-1, 1], "bin_index": 0}]}]}]}
    path = tmp_path / "m.json"
    path.write_text(json.dumps(m))
    iv = gp.load_range_label_manifest(str(path), 6)
    assert iv.range_count == 2
    assert iv.has_interval.tolist() == [0, 0, 1, 1, 0, 1]
    assert iv.range_index[5] == 1 and iv.bin[3] == 1 and iv.lower[5] == -1
    lay = gp.build_range_cover_layout(iv, 1)
    assert gp.plan_pure_range_cover(lay, 3, -0.5, 0.5) == [5]
    assert gp.plan_pure_range_cover(gp.build_range_cover_layout(iv, 0), 1, 5, 0) == [2, 3]
    m["ranges"][0]["levels"][0]["partitions"][0]["label_id"] = 9
    path.write_text(json.dumps(m))
    with pytest.raises(ValueError, match="label_id out of range"):
        gp.load_range_label_manifest(str(path), 6)


def test_cover_gap_is_an_error(tmp_path):
    # a missing finest bin inside the target leaves a gap
    levels = [{"level_index": 0, "partitions": [
        {"label_id": 0, "interval": [0, 1], "bin_index": 0},
        {"label_id": 2, "interval": [2, 3], "bin_index": 2}]}]
    path = tmp_path / "m.json"
    path.write_text(json.dumps({"levels": levels}))
    lay = gp.build_range_cover_layout(gp.load_range_label_manifest(str(path), 3), 0)
    assert gp.plan_pure_range_cover(lay, 3, 0.0, 0.9) == [0]
    with pytest.raises(ValueError, match="gap"):
        gp.plan_pure_range_cover(lay, 3, 0.5, 2.5)
