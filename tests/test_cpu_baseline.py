"""The CPU baseline (oracle/libgofann_cpu_baseline.so: the oracle's batch
drivers over host cores with OpenMP, -O3) returns exactly what the
single-threaded oracle returns: ids, distance bits and counters, for every
driver the bench times."""
from __future__ import annotations

import numpy as np
import pytest

import pyoracle as po
from gofann_amd import index as gi
from gofann_amd import plan as gp
from gofann_amd import synth

# the index is built by the oracle's restatement of the GPU build (no GPU here)
CPU_BUILD = po.OracleBuild()


@pytest.fixture(scope="module")
def world():
    wl = synth.small_labelled(n=5000, nq=70, dim=32, k=8, sigma=0.7, labels=5, seed=41,
                              tags=True, ranges=True, dtype="u8")
    cen = gi.train_kmeans(wl.base, 8, seed=41, backend=CPU_BUILD)
    li = gi.build_label_index(wl.base, wl.label_offsets, wl.label_values, wl.num_labels, cen,
                              degree=32, threshold=150, backend=CPU_BUILD)
    pl = gp.plan_queries(li, wl.query_labels, wl.query_ranges)
    assert pl.graph.count > 40
    return wl, li, pl, cen


def _same(a, b):
    for x, y in zip(a, b):
        x, y = np.asarray(x), np.asarray(y)
        assert x.dtype == y.dtype and x.shape == y.shape
        assert np.array_equal(x.view(np.uint8), y.view(np.uint8))


@pytest.mark.parametrize("threads", [1, 3, 8])
def test_exact_search_threads_identical(world, threads):
    wl, li, pl, _ = world
    rs = pl.graph
    pred = po.PredicateArrays.from_plan(rs.predicate, li, wl.base_ranges)
    args = (li, rs, pred, wl.base.numpy(), wl.queries.numpy())
    kw = dict(queue_limit=48, topk=10, label_size=li.label_size)
    _same(po.exact_search(*args, **kw), po.exact_search(*args, **kw, threads=threads))


@pytest.mark.parametrize("inline", [False, True])
def test_pq_search_threads_identical(world, inline):
    wl, li, pl, _ = world
    rs = pl.graph
    table = gi.train_pq(wl.base, 8, iters=4, backend=CPU_BUILD)
    codes = gi.pq_encode(wl.base, table, 8, backend=CPU_BUILD).numpy()
    pred = po.PredicateArrays.from_plan(rs.predicate, li, wl.base_ranges, alpha=0.15,
                                        pending_base_stop=True)
    prm = po.params(queue_limit=40, result_width=10 if inline else 30, inline_exact=inline)
    base = wl.base.numpy() if inline else None
    a = po.pq_search(li, rs, pred, prm, codes, table.numpy(), wl.queries.numpy(), base=base)
    b = po.pq_search(li, rs, pred, prm, codes, table.numpy(), wl.queries.numpy(), base=base,
                     threads=5)
    _same(a, b)
    pr = po.PredicateArrays.from_plan(pl.posting.predicate, li, wl.base_ranges)
    if pl.posting.count:
        args = (pr, codes, table.numpy(), wl.queries.numpy(), pl.posting.route_query,
                li.posting_ids, pl.cand_offsets, pl.cand_sizes, 20)
        _same(po.posting_scan_pq(*args), po.posting_scan_pq(*args, threads=4))


def test_rabitq_drivers_threads_identical(world):
    wl, li, pl, cen = world
    rs = pl.graph
    P = 64
    x = wl.base.float()
    rot = gi.random_rotation(wl.dim, P, 41, "cpu")
    codes, fac, aid, anchors = gi.rabitq_encode(x, rot, cen, backend=CPU_BUILD)
    qr = (wl.queries.float() @ rot).numpy()
    nq = qr.shape[0]
    q8 = np.empty((nq, P), np.int8)
    sc = np.empty(nq, np.float32)
    k1 = np.empty(nq, np.float32)
    for i in range(nq):
        q8[i], sc[i], k1[i] = po.rabitq_quantize(qr[i])
    an = anchors.numpy().astype(np.float64)
    cd = ((qr.astype(np.float64)[:, None, :] - an[None]) ** 2).sum(-1).astype(np.float32)
    pred = po.PredicateArrays.from_plan(rs.predicate, li, wl.base_ranges, alpha=0.15,
                                        pending_base_stop=True)
    prm = po.params(queue_limit=32, result_width=20, rabitq_verdict=1)
    args = (li, rs, pred, prm, codes.numpy(), fac.numpy(), aid.numpy().astype(np.uint32), q8, sc,
            k1, cd, anchors.shape[0], P)
    _same(po.rabitq_search(*args), po.rabitq_search(*args, threads=6))
    # label posting scan over every route's group posting list
    ga = rs.route_group
    offs = li.posting_offset[ga].astype(np.uint32)
    sizes = (li.posting_offset[ga + 1] - li.posting_offset[ga]).astype(np.uint32)
    args = (pred, codes.numpy(), fac.numpy(), aid.numpy().astype(np.uint32), q8, sc, k1, cd,
            rs.route_query, li.posting_ids, offs, sizes, 15)
    _same(po.posting_scan_rabitq(*args), po.posting_scan_rabitq(*args, threads=3))
    # range posting scan in segments
    order = np.argsort(wl.base_ranges[:, 0], kind="stable").astype(np.uint32)
    nseg = 40
    seg_routes = (np.arange(nseg) % rs.count).astype(np.uint32)
    seg_off = (np.arange(nseg) * 97 % wl.n).astype(np.uint64)
    seg_size = np.full(nseg, 300, np.uint64)
    modes = np.full((rs.count, 1), 3, np.uint8)
    lo = np.full((rs.count, 1), 100, np.float32)
    hi = np.full((rs.count, 1), 700, np.float32)
    args = (pred, modes, lo, hi, wl.base_ranges, codes.numpy(), fac.numpy(),
            aid.numpy().astype(np.uint32), q8, sc, k1, cd, rs.route_query, order, wl.n, wl.n,
            seg_routes, seg_off, seg_size, 25)
    _same(po.rabitq_range_scan(*args), po.rabitq_range_scan(*args, threads=4))


def test_rerank_threads_identical(world):
    wl, li, pl, _ = world
    rng = np.random.default_rng(2)
    rq = rng.integers(0, wl.queries.shape[0], 300).astype(np.uint32)
    sl = rng.integers(0, wl.n, (300, 40)).astype(np.uint32)
    sl[::7, 5] = 0xFFFFFFFF
    for base, q in ((wl.base.numpy(), wl.queries.numpy()),
                    (wl.base.numpy().astype(np.float32), wl.queries.numpy().astype(np.float32)),
                    (wl.base.numpy().astype(np.float16), wl.queries.numpy().astype(np.float32))):
        _same(po.rerank(base, q, rq, sl, 10), po.rerank(base, q, rq, sl, 10, threads=4))
