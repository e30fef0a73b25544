"""Pins the oracle traversal by brute force: with a beam at least as large as
a label group and early stop off, the label-partitioned beam search visits
the whole (connected) group, so its W results must be exactly the W best
predicate-passing rows by the same distance, in (distance, pop) order."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import pyoracle as po
from gofann_amd import index as gi
from gofann_amd import plan as gp
from gofann_amd import synth

# the index is built by the oracle's restatement of the GPU build (no GPU here)
CPU_BUILD = po.OracleBuild()

U32MAX = 0xFFFFFFFF


@pytest.fixture(scope="module")
def tiny():
    wl = synth.small_labelled(n=900, nq=12, dim=32, k=6, sigma=0.8, labels=3, seed=5, tags=True)
    li = gi.build_label_index(wl.base, wl.label_offsets, wl.label_values, wl.num_labels,
                              wl.centroids, degree=24, threshold=50,
                              backend=CPU_BUILD)
    table = gi.train_pq(wl.base, 8, iters=8, backend=CPU_BUILD)
    codes = gi.pq_encode(wl.base, table, 8, backend=CPU_BUILD)
    pl = gp.plan_queries(li, wl.query_labels)
    return wl, li, table.numpy(), codes.numpy(), pl


def _adc_all(table, codes, q, M):
    lut = po.pq_lut(table, q, M)
    return np.array([po.pq_adc(lut, codes[s]) for s in range(codes.shape[0])], np.float32)


def complete_graph_index(wl, group_cap=60):
    """Same labels, but each label group keeps its first `group_cap` samples
    and its graph is complete (every row lists every other row).  The beam
    then scores the whole group from the seed, and the one node the drained
    loop leaves unexpanded is the farthest, so the top W (W < group size - 1)
    are exactly the brute-force W best passing rows."""
    li = gi.build_label_index(wl.base, wl.label_offsets, wl.label_values, wl.num_labels,
                              wl.centroids, degree=64, threshold=50,
                              backend=CPU_BUILD)
    sizes = np.minimum(li.label_size, group_cap).astype(np.uint32)
    offs = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.uint32)
    r2s = np.concatenate([li.row_to_sample[li.label_offset[l]:li.label_offset[l] + sizes[l]]
                          for l in range(li.num_labels)]).astype(np.uint32)
    graph = np.full((len(r2s), 64), U32MAX, np.uint32)
    for l in range(li.num_labels):
        n = int(sizes[l])
        for i in range(n):
            nb = [j for j in range(n) if j != i]
            graph[offs[l] + i, :len(nb)] = nb
    li.label_size, li.label_offset, li.row_to_sample, li.graph = sizes, offs, r2s, graph
    li.seed_local = np.where(sizes > 0, 0, U32MAX).astype(np.uint32)
    return li


@pytest.mark.parametrize("bias", [False, True])
def test_full_beam_equals_brute_force(tiny, bias):
    wl, _, table, codes, _ = tiny
    li = complete_graph_index(wl)
    rs = gp.plan_queries(li, wl.query_labels).graph
    W = 8
    pred = po.PredicateArrays.from_plan(rs.predicate, li, alpha=0.15 if bias else 0.0,
                                        pending_base_stop=bias)
    prm = po.params(queue_limit=1000, result_width=W, early_stop_mode=1, bias=bias)
    q = wl.queries.numpy()
    ids, dists, st = po.pq_search(li, rs, pred, prm, codes, table, q)
    M = codes.shape[1]
    for r in range(rs.count):
        label = int(rs.route_group[r])
        qi = int(rs.route_query[r])
        rows = li.row_to_sample[li.label_offset[label]:li.label_offset[label] + li.label_size[label]]
        allowed = gp.filter_mask(li, wl.query_labels[qi], [], None)
        cand = np.array([s for s in rows if allowed[s]], dtype=np.int64)
        d = _adc_all(table, codes, q[qi], M)
        order = sorted(zip(d[cand].tolist(), cand.tolist()))[:W]
        got = [(float(x), int(i)) for x, i in zip(dists[r], ids[r]) if i != U32MAX]
        assert sorted(got) == sorted(order), r
        assert all(got[i][0] <= got[i + 1][0] for i in range(len(got) - 1))
        assert st[r, 7] == 1  # the beam ran dry (no early stop)
        # every row but the one held when the pool ran dry is expanded once
        # (backend_pq.cu:4451-4461); the seed plus every other row is scored
        assert st[r, 1] == len(rows) - 1
        assert st[r, 3] == len(rows) and st[r, 6] == len(rows) - 1


def test_adaptive_stop_recall(tiny):
    wl, li, table, codes, pl = tiny
    rs = pl.graph
    pred = po.PredicateArrays.from_plan(rs.predicate, li, alpha=0.15, pending_base_stop=True)
    full = po.params(queue_limit=1000, result_width=10, early_stop_mode=1)
    fast = po.params(queue_limit=32, result_width=10, early_stop_mode=2)
    q = wl.queries.numpy()
    a, _, sa = po.pq_search(li, rs, pred, full, codes, table, q)
    b, _, sb = po.pq_search(li, rs, pred, fast, codes, table, q)
    hit = np.mean([len(set(a[r]) & set(b[r]) - {U32MAX}) / max(1, len(set(a[r]) - {U32MAX}))
                   for r in range(rs.count)])
    assert hit >= 0.75  # early stop keeps most of the full-beam answer
    assert sb[:, 0].sum() < sa[:, 0].sum()


def test_max_steps_and_stats_consistency(tiny):
    wl, li, table, codes, pl = tiny
    rs = pl.graph
    pred = po.PredicateArrays.from_plan(rs.predicate, li, alpha=0.15, pending_base_stop=True)
    prm = po.params(queue_limit=16, result_width=10, early_stop_mode=1, max_steps=5)
    _, _, st = po.pq_search(li, rs, pred, prm, codes, table, wl.queries.numpy())
    assert np.all(st[:, 0] <= 5) and np.all(st[:, 1] <= 4)
    assert np.all(st[:, 2] <= st[:, 1])
    assert np.all(st[:, 3] >= 1 + st[:, 6])  # scored >= seed + admitted


def test_oracle_rabitq_full_beam(tiny):
    wl = tiny[0]
    li = complete_graph_index(wl)
    rs = gp.plan_queries(li, wl.query_labels).graph
    x = wl.base
    P = 64
    rot = gi.random_rotation(x.shape[1], P, 5, "cpu")
    rcodes, fac, aid, anchors = gi.rabitq_encode(x, rot, wl.centroids, backend=CPU_BUILD)
    qr = (wl.queries.float() @ rot).numpy()
    nq = qr.shape[0]
    q8 = np.empty((nq, P), np.int8)
    sc = np.empty(nq, np.float32)
    k1 = np.empty(nq, np.float32)
    for i in range(nq):
        q8[i], sc[i], k1[i] = po.rabitq_quantize(qr[i])
    an = anchors.numpy().astype(np.float64)
    cd = ((qr.astype(np.float64)[:, None, :] - an[None]) ** 2).sum(-1).astype(np.float32)
    W = 8
    pred = po.PredicateArrays.from_plan(rs.predicate, li, alpha=0.15, pending_base_stop=True)
    prm = po.params(queue_limit=1000, result_width=W, early_stop_mode=1, rabitq_verdict=1)
    ids, dists, st = po.rabitq_search(li, rs, pred, prm, rcodes.numpy(), fac.numpy(),
                                      aid.numpy().astype(np.uint32), q8, sc, k1, cd,
                                      anchors.shape[0], P)
    L = po.lib()
    for r in range(rs.count):
        label = int(rs.route_group[r])
        qi = int(rs.route_query[r])
        rows = li.row_to_sample[li.label_offset[label]:li.label_offset[label] + li.label_size[label]]
        allowed = gp.filter_mask(li, wl.query_labels[qi], [], None)
        cand = [int(s) for s in rows if allowed[s]]
        est = []
        for s in cand:
            ip = po.rabitq_ip(q8[qi], rcodes.numpy()[s], "int")
            est.append(L.orc_rabitq_score_b1(ip, sc[qi], k1[qi], fac[s, 0].item(), fac[s, 1].item(),
                                             cd[qi, int(aid[s])]))
        want = sorted(zip(np.array(est, np.float32).tolist(), cand))[:W]
        got = [(float(a), int(b)) for a, b in zip(dists[r], ids[r]) if b != U32MAX]
        assert sorted(got) == sorted(want)


@pytest.mark.parametrize("bias", [False, True])
def test_inline_exact_full_beam_equals_exact_brute_force(tiny, bias):
    """Inline exact ranking (backend_pq.cu:4507-4546): the result heap is
    ordered by the true L2 distance of each expanded passing row.  With the
    complete-graph group every row but one is expanded, so the W results
    are the W exactly-nearest passing rows of the group with at most one
    row left out, and every returned distance is that row's exact L2."""
    wl, _, table, codes, _ = tiny
    li = complete_graph_index(wl)
    rs = gp.plan_queries(li, wl.query_labels).graph
    W = 8
    pred = po.PredicateArrays.from_plan(rs.predicate, li, alpha=0.15 if bias else 0.0,
                                        pending_base_stop=bias)
    prm = po.params(queue_limit=1000, result_width=W, early_stop_mode=1, bias=bias,
                    inline_exact=True)
    q = wl.queries.numpy()
    base = wl.base.numpy()
    ids, dists, st = po.pq_search(li, rs, pred, prm, codes, table, q, base=base)
    for r in range(rs.count):
        label = int(rs.route_group[r])
        qi = int(rs.route_query[r])
        rows = li.row_to_sample[li.label_offset[label]:li.label_offset[label] + li.label_size[label]]
        allowed = gp.filter_mask(li, wl.query_labels[qi], [], None)
        cand = [int(s) for s in rows if allowed[s]]
        exact = {s: float(((base[s].astype(np.float64) - q[qi]) ** 2).sum()) for s in cand}
        got = [(float(d), int(i)) for d, i in zip(dists[r], ids[r]) if i != U32MAX]
        for d, i in got:
            assert d == pytest.approx(exact[i], rel=1e-5, abs=1e-4)
        assert all(got[k][0] <= got[k + 1][0] for k in range(len(got) - 1))
        ranked = sorted(cand, key=lambda s: (exact[s], s))
        got_ids = [i for _, i in got]
        options = [ranked[:W]] + [[s for s in ranked if s != x][:W] for x in ranked[:W]]
        assert any(sorted(got_ids) == sorted(o) for o in options), r
        assert st[r, 2] >= len(cand) - 1


def test_inline_exact_u8_distances_are_integer_exact():
    """uint8 inline exact: each lane's squared differences are integers and
    their float sums stay below 2^24, so every distance is the exact integer
    squared L2."""
    wl = synth.small_labelled(n=700, nq=8, dim=48, k=5, sigma=0.8, labels=2, seed=9, tags=True,
                              dtype="u8")
    li = gi.build_label_index(wl.base, wl.label_offsets, wl.label_values, wl.num_labels,
                              wl.centroids, degree=16, threshold=40,
                              backend=CPU_BUILD)
    table = gi.train_pq(wl.base, 8, iters=6, backend=CPU_BUILD)
    codes = gi.pq_encode(wl.base, table, 8, backend=CPU_BUILD)
    rs = gp.plan_queries(li, wl.query_labels).graph
    pred = po.PredicateArrays.from_plan(rs.predicate, li, alpha=0.15, pending_base_stop=True)
    prm = po.params(queue_limit=64, result_width=10, inline_exact=True)
    q = wl.queries.numpy()
    base = wl.base.numpy()
    ids, dists, _ = po.pq_search(li, rs, pred, prm, codes.numpy(), table.numpy(), q, base=base)
    n_checked = 0
    for r in range(rs.count):
        for d, i in zip(dists[r], ids[r]):
            if i == U32MAX:
                continue
            want = int(((base[i].astype(np.int64) - q[rs.route_query[r]].astype(np.int64)) ** 2)
                       .sum())
            assert float(d) == float(want)
            n_checked += 1
    assert n_checked > 0
