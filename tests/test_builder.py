"""Host-side index building (the orchestration of gofann_amd.index over the
oracle's restatement of the GPU build primitives) and the C3 workload
generator.  CPU only."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import pyoracle as po
from gofann_amd import index as gi
from gofann_amd import synth

U32MAX = 0xFFFFFFFF
CPU_BUILD = po.OracleBuild()


@pytest.mark.parametrize("design", ["navigable", "cagra"])
def test_label_graphs_deterministic_and_well_formed(design):
    """Two builds from the same inputs are identical; every row's links are
    distinct rows of its own group other than itself; the seed is the
    group's medoid; the entry row links to `degree` distinct rows; with the
    cagra design every row is reachable from the seed (the repair's
    guarantee)."""
    wl = synth.small_labelled(n=2400, nq=4, dim=24, k=10, sigma=0.6, labels=3, seed=7)
    cen = gi.train_kmeans(wl.base, 12, seed=3, backend=CPU_BUILD)
    args = (wl.base, wl.label_offsets, wl.label_values, wl.num_labels, cen)
    a = gi.build_label_index(*args, degree=16, threshold=100, design=design, backend=CPU_BUILD)
    b = gi.build_label_index(*args, degree=16, threshold=100, design=design, backend=CPU_BUILD)
    assert np.array_equal(a.graph, b.graph) and np.array_equal(a.seed_local, b.seed_local)
    base = wl.base.numpy()
    for l in np.nonzero(a.label_size)[0]:
        o, m = int(a.label_offset[l]), int(a.label_size[l])
        g = a.graph[o:o + m]
        for i in range(m):
            row = g[i][g[i] != U32MAX]
            assert len(set(row.tolist())) == len(row) and np.all(row < m) and i not in row
        samples = a.row_to_sample[o:o + m]
        xg = base[samples].astype(np.float64)
        assert a.seed_local[l] == int(((xg - xg.mean(0)) ** 2).sum(1).argmin())
        entry = g[a.seed_local[l]]
        assert np.all(entry != U32MAX) and len(set(entry.tolist())) == 16
        if design == "cagra":
            reached, cnt = po.build_reach(g, int(a.seed_local[l]))
            assert cnt == m


def test_navigable_links_hold_the_bucket_knn_prefix():
    """An ordinary row of the navigable design starts with its exact
    in-bucket nearest rows (gofann_build_knn over the bucket-sorted rows),
    mapped back to the group's row order."""
    wl = synth.small_labelled(n=1500, nq=4, dim=16, k=6, sigma=0.6, labels=1, seed=9)
    cen = gi.train_kmeans(wl.base, 6, seed=2, backend=CPU_BUILD)
    li = gi.build_label_index(wl.base, wl.label_offsets, wl.label_values, wl.num_labels, cen,
                              degree=12, threshold=10, local=5, backend=CPU_BUILD)
    l = int(np.nonzero(li.label_size)[0][0])
    o, m = int(li.label_offset[l]), int(li.label_size[l])
    samples = li.row_to_sample[o:o + m]
    x = wl.base.numpy()[samples]
    cl = po.build_assign(x, cen.numpy())[0].astype(np.int64)
    order, uniq, off, bucket_of = gi._bucket_order(cl)
    knn, _ = po.build_knn(x[order], off, 5)
    reps = set(li.rep_row.tolist())
    checked = 0
    for s in range(m):
        i = order[s]
        if i in reps or i == li.seed_local[l]:
            continue
        want = [int(order[v]) for v in knn[s] if v != U32MAX][:5]
        assert li.graph[o + i][:len(want)].tolist() == want
        checked += 1
    assert checked > m // 2


def test_train_kmeans_is_seeded_and_deterministic():
    x = torch.from_numpy(np.random.default_rng(4).standard_normal((3000, 8)).astype(np.float32))
    a = gi.train_kmeans(x, 16, iters=5, sample=2000, seed=11, backend=CPU_BUILD)
    b = gi.train_kmeans(x, 16, iters=5, sample=2000, seed=11, backend=CPU_BUILD)
    c = gi.train_kmeans(x, 16, iters=5, sample=2000, seed=12, backend=CPU_BUILD)
    assert torch.equal(a, b) and not torch.equal(a, c)
    # every centre is the mean of its sample rows after the last iteration
    idx = gi._sample(3000, 2000, 11)
    xs = x.numpy()[idx]
    prev = gi.train_kmeans(x, 16, iters=4, sample=2000, seed=11, backend=CPU_BUILD).numpy()
    assign = po.build_assign(xs, prev)[0]
    for k in range(16):
        rows = xs[assign == k]
        if len(rows):
            assert np.array_equal(a[k].numpy(),
                                  (rows.astype(np.float64).sum(0) / len(rows)).astype(np.float32))


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
