"""Host-side index building and the C3 workload generator (CPU only)."""
from __future__ import annotations

import numpy as np
import torch

from gofann_amd import index as gi
from gofann_amd import synth


def test_lean_group_builder_matches_default(monkeypatch):
    """Large groups are built without full row copies (rows gathered per
    bucket batch, means, distances and the fp64 seed a chunk at a time); the
    graph, representatives and seeds must equal the copying build's."""
    wl = synth.config3(n=3000, nq=8, device="cpu", dim=64, k=16, rank=8, seed=5)
    args = (wl.base, wl.label_offsets, wl.label_values, wl.num_labels, wl.centroids)
    ref = gi.build_label_index(*args, degree=16, threshold=100)
    monkeypatch.setattr(gi, "LEAN_GROUP_BYTES", 0)
    lean = gi.build_label_index(*args, degree=16, threshold=100)
    assert np.array_equal(ref.graph, lean.graph)
    assert np.array_equal(ref.row_to_sample, lean.row_to_sample)
    assert np.array_equal(ref.seed_local, lean.seed_local)


def test_config3_shapes_and_ranges():
    wl = synth.config3(n=4000, nq=30, device="cpu", dim=32, k=8, rank=4, seed=2)
    assert wl.base.shape == (4000, 32) and wl.queries.shape == (30, 32)
    assert torch.allclose(wl.base.norm(dim=1), torch.ones(4000), atol=1e-5)
    attr = wl.base_ranges[:, 0]
    assert attr.min() >= 0 and attr.max() < 10_000 and np.all(attr == np.floor(attr))
    sel = wl.meta["selectivity"]
    for i, rr in enumerate(wl.query_ranges):
        (col, mode, lo, hi), = rr
        assert col == 0 and mode == 3 and 0 <= lo and hi <= 10_000
        assert hi - lo == max(1, round(sel[i] * 10_000))
    # one group holding every row, in sample order
    assert wl.num_labels == 1 and np.array_equal(wl.label_offsets, np.arange(4001))
