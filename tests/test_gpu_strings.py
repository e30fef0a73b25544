"""GPU parity of the C5 route set: a small world with category, range and
string-token labels, every query a DNF filter (exact string, fuzzy string
expanded over 3-gram Jaccard, category AND range AND string), planned into
graph routes and label-posting routes (clause scans included).  The RaBitQ
traversal of the graph routes and the segmented label-posting scan with
posting-order columns equal the oracle's, ids, distance bits and counters."""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import pyoracle as po
from gofann_amd import _lib
from gofann_amd import index as gi
from gofann_amd import plan as gp
from gofann_amd import range_posting as rp
from gofann_amd import search as gs
from gofann_amd import synth

pytestmark = pytest.mark.gpu
U32MAX = 0xFFFFFFFF


def say(*a):
    print("[gpu-test]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def c5():
    wl = synth.config5(n=40_000, nq=120, device="cpu", dim=64, k=32, labels=20, intervals=10,
                       vocab=500)
    cen = gi.train_kmeans(wl.base, 32, seed=4)
    li = gi.build_label_index(wl.base.float(), wl.label_offsets, wl.label_values, wl.num_labels,
                              cen, degree=32, threshold=700, local=12)
    P = 128
    rot = gi.random_rotation(wl.dim, P, 5, "cpu")
    codes, fac, aid, anchors = gi.rabitq_encode(wl.base.float(), rot, cen)
    return wl, li, P, rot, codes, fac, aid, anchors


def test_c5_routes_match_oracle(gpu_ctx, c5):
    wl, li, P, rot, codes, fac, aid, anchors = c5
    g_rows, p_rows = gp.dnf_route_rows(li, wl.meta["query_clauses"], wl.query_ranges,
                                       clause_scans=True)
    rs, ps = gp._routeset(g_rows, li), gp._routeset(p_rows, li)
    say("c5 routes", rs.count, ps.count)
    assert rs.count > 50 and ps.count > 50
    dev = dict(codes=codes.cuda(), fac=fac.cuda(), aid=aid.cuda(), anchors=anchors.cuda(),
               rot=rot.cuda(), q=wl.queries.float().cuda())
    rv = _lib.RabitqView(_lib.ptr(dev["codes"]), _lib.ptr(dev["fac"]), _lib.ptr(dev["aid"]),
                         _lib.ptr(dev["anchors"]), wl.dim, P, anchors.shape[0], wl.n)
    nq = wl.queries.shape[0]
    A = anchors.shape[0]
    prep = dict(rotated=torch.empty(nq, P, device="cuda"),
                q8=torch.empty(nq, P, dtype=torch.int8, device="cuda"),
                scale=torch.empty(nq, device="cuda"), k1=torch.empty(nq, device="cuda"),
                cd=torch.empty(nq, A, device="cuda"))
    rq = _lib.RabitqQueries(*[_lib.ptr(prep[k]) for k in ("rotated", "q8", "scale", "k1", "cd")],
                            nq)
    gpu_ctx.check(gpu_ctx.lib.gofann_rabitq_prepare_queries(gpu_ctx.handle, rv, _lib.ptr(dev["q"]),
                                                            nq, _lib.ptr(dev["rot"]), rq))
    torch.cuda.synchronize()
    h = {k: v.cpu().numpy() for k, v in prep.items()}
    W = 50
    # graph routes: RaBitQ traversal with each route's DNF residual
    dg = gs.DeviceGraph.upload(li)
    dr = gs.DeviceRoutes.upload(rs, wl.base_ranges)
    prm = gs.search_params(queue_limit=96, result_width=W, early_stop_mode=2, bias=True)
    n = rs.count
    ids = torch.empty(n * W, dtype=torch.int32, device="cuda")
    dists = torch.empty(n * W, device="cuda")
    stats = torch.zeros(n * 8, dtype=torch.int32, device="cuda")
    gpu_ctx.check(gpu_ctx.lib.gofann_rabitq_search(
        gpu_ctx.handle, rv, rq, dg.view(), dr.predicate_view(dg, 0.15, True), dr.routes_view(),
        prm, _lib.ptr(ids), _lib.ptr(dists), _lib.ptr(stats)))
    torch.cuda.synchronize()
    pg = po.PredicateArrays.from_plan(rs.predicate, li, base_ranges=wl.base_ranges, alpha=0.15,
                                      pending_base_stop=True)
    oi, od, ost = po.rabitq_search(li, rs, pg, po.params(queue_limit=96, result_width=W,
                                                         early_stop_mode=2, bias=True,
                                                         rabitq_verdict=1),
                                   codes.numpy(), fac.numpy(), aid.numpy().astype(np.uint32),
                                   h["q8"], h["scale"], h["k1"], h["cd"], A, P, threads=4)
    assert np.array_equal(ids.cpu().numpy().view(np.uint32).reshape(n, W), oi)
    assert np.array_equal(dists.cpu().numpy().reshape(n, W).view(np.uint32), od.view(np.uint32))
    assert np.array_equal(stats.cpu().numpy().reshape(n, 8), ost)
    # posting routes: segmented scan over posting-order columns
    m = ps.count
    off = np.array([li.posting_offset[r[1]] for r in p_rows], np.uint64)
    size = np.array([li.posting_offset[r[1] + 1] - li.posting_offset[r[1]] for r in p_rows],
                    np.uint64)
    dp = gs.DeviceRoutes.upload(ps, wl.base_ranges)
    pv = dp.predicate_view(dg, 0.0, False)
    total = int(li.posting_offset[-1])
    segs = rp.DeviceSegments(rp.segment_plan(np.arange(m), off, size, 512))
    rows = rp.PostingRows(gpu_ctx, rv, dg.posting_ids, total)
    cols = rp.PostingPredicateColumns(gpu_ctx, pv, dg.posting_ids, total)
    pi, pd, pp = rp.rabitq_posting_scan_segments(gpu_ctx, rv, rq, pv, dp.route_query,
                                                 dg.posting_ids, total, segs, W, rows=rows,
                                                 cols=cols)
    torch.cuda.synchronize()
    pr = po.PredicateArrays.from_plan(ps.predicate, li, base_ranges=wl.base_ranges)
    qi, qd, qp = po.posting_scan_rabitq(pr, codes.numpy(), fac.numpy(),
                                        aid.numpy().astype(np.uint32), h["q8"], h["scale"],
                                        h["k1"], h["cd"], ps.route_query, li.posting_ids,
                                        off.astype(np.uint32), size.astype(np.uint32), W)
    assert np.array_equal(pi.cpu().numpy().view(np.uint32), qi)
    assert np.array_equal(pd.cpu().numpy().view(np.uint32), qd.view(np.uint32))
    assert np.array_equal(pp.cpu().numpy().view(np.uint32), qp)
    assert (qi[:, 0] != U32MAX).sum() > m // 2
    # the label-shared scan (the routes of a label share each segment's rows)
    if W <= 128:
        share = rp.DeviceShare(rp.share_plan(segs.plan))
        si, sd, spp = rp.rabitq_posting_scan_segments(gpu_ctx, rv, rq, pv, dp.route_query,
                                                      dg.posting_ids, total, segs, W, rows=rows,
                                                      cols=cols, share=share)
        torch.cuda.synchronize()
        assert np.array_equal(si.cpu().numpy().view(np.uint32), qi)
        assert np.array_equal(sd.cpu().numpy().view(np.uint32), qd.view(np.uint32))
        assert np.array_equal(spp.cpu().numpy().view(np.uint32), qp)
