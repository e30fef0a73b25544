"""GPU parity of the RaBitQ range-posting scan and segment merge: the HIP
kernels behind gofann_rabitq_range_scan against the oracle on the same
prepared queries, bit-exact (ids, distance bits, pass counts), over shortlist
sizes that take every merge path (k = 10 .. 4096), unsegmented and segmented
plans, filter-first and score-first, with and without a device predicate."""
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


def as_u32(t):
    return t.cpu().numpy().view(np.uint32)


# Padded dims: 128 .. 4096 take the group-per-row kernel with groups of
# 1 .. 32 lanes, 8192 its two-vectors-per-lane form, 384 (three 16-byte
# vectors) the thread-per-row kernel.
@pytest.fixture(scope="module", params=[128, 384, 1024, 4096, 8192])
def rangeworld(request, gpu_ctx):
    wl = synth.small_labelled(n=6000, nq=40, dim=60, k=10, sigma=0.7, labels=5, seed=41, tags=True)
    li = gi.build_label_index(wl.base, wl.label_offsets, wl.label_values, wl.num_labels,
                              wl.centroids, degree=32, threshold=300)
    P = request.param
    say("range world, padded dim", P)
    if P <= 1024:
        rot = gi.random_rotation(wl.dim, P, 41005, "cpu")
    else:
        # any [dim][P] matrix gives codes both sides score alike; a QR this
        # large would dominate the test
        g = torch.Generator().manual_seed(41005)
        rot = torch.randn(wl.dim, P, generator=g) / P ** 0.5
    codes, fac, aid, anchors = gi.rabitq_encode(wl.base, rot, wl.centroids)
    n = wl.n
    rng = np.random.default_rng(41)
    rc = 2
    base_ranges = rng.integers(0, 50, (n, rc)).astype(np.float32)   # many equal values
    routes = 48
    route_query = rng.integers(0, wl.queries.shape[0], routes).astype(np.uint32)
    modes = rng.integers(0, 4, (routes, rc)).astype(np.uint8)
    modes[0] = 0                                   # no active range: empty output
    modes[1] = [3, 3]
    modes[2] = [1, 0]                              # a long slice (values > lower)
    lower = rng.integers(0, 30, (routes, rc)).astype(np.float32)
    upper = lower + rng.integers(5, 40, (routes, rc)).astype(np.float32)
    lower[2, 0] = 2.0
    index = rp.RangePostingIndex.build(base_ranges)
    slices = rp.choose_slices(index, modes, lower, upper)
    offsets, sizes = rp.route_postings(index, slices)
    # residual predicate: the query's labels and its range atoms
    rows = []
    for r in range(routes):
        labels = wl.query_labels[int(route_query[r])][:1] if r % 3 else []
        rng_atoms = [(d, int(modes[r, d]), float(lower[r, d]), float(upper[r, d]))
                     for d in range(rc) if modes[r, d]]
        rows.append((int(route_query[r]), 0, labels, rng_atoms))
    rs = gp._routeset(rows, li)

    dev = dict(codes=codes.cuda(), fac=fac.cuda(), aid=aid.cuda(), anchors=anchors.cuda(),
               rot=rot.cuda(), q=wl.queries.float().cuda())
    rv = _lib.RabitqView(_lib.ptr(dev["codes"]), _lib.ptr(dev["fac"]), _lib.ptr(dev["aid"]),
                         _lib.ptr(dev["anchors"]), wl.dim, P, anchors.shape[0], n)
    nq = wl.queries.shape[0]
    A = anchors.shape[0]
    out = dict(rotated=torch.empty(nq, P, device="cuda"),
               q8=torch.empty(nq, P, dtype=torch.int8, device="cuda"),
               scale=torch.empty(nq, device="cuda"), k1=torch.empty(nq, device="cuda"),
               cd=torch.empty(nq, A, device="cuda"))
    rq = _lib.RabitqQueries(_lib.ptr(out["rotated"]), _lib.ptr(out["q8"]), _lib.ptr(out["scale"]),
                            _lib.ptr(out["k1"]), _lib.ptr(out["cd"]), nq)
    gpu_ctx.check(gpu_ctx.lib.gofann_rabitq_prepare_queries(gpu_ctx.handle, rv, _lib.ptr(dev["q"]), nq,
                                                            _lib.ptr(dev["rot"]), rq))
    torch.cuda.synchronize()
    host_q = {k: v.cpu().numpy() for k, v in out.items()}
    dev["prepared"] = out  # rq holds raw pointers into these tensors
    dg = gs.DeviceGraph.upload(li)
    dr = gs.DeviceRoutes.upload(rs, base_ranges)
    dev.update(postings=index.device_postings(), modes=torch.from_numpy(modes).cuda(),
               lower=torch.from_numpy(lower).cuda(), upper=torch.from_numpy(upper).cuda(),
               brv=torch.from_numpy(base_ranges).cuda(),
               rquery=torch.from_numpy(route_query.view(np.int32)).cuda())
    return dict(wl=wl, li=li, codes=codes.numpy(), fac=fac.numpy(), aid=aid.numpy().astype(np.uint32),
                P=P, A=A, rv=rv, rq=rq, host_q=host_q, index=index, modes=modes, lower=lower,
                upper=upper, base_ranges=base_ranges, route_query=route_query, offsets=offsets,
                sizes=sizes, rs=rs, dg=dg, dr=dr, dev=dev, routes=routes)


def _routes_view(w):
    d = w["dev"]
    return _lib.Routes(_lib.ptr(d["rquery"]), None, None, None, None, _lib.ptr(d["modes"]),
                       _lib.ptr(d["lower"]), _lib.ptr(d["upper"]), _lib.ptr(d["brv"]), 2,
                       w["routes"], None)


def _oracle(w, pred, seg_routes, seg_off, seg_size, k, score_first, resident=None):
    hq = w["host_q"]
    return po.rabitq_range_scan(pred, w["modes"], w["lower"], w["upper"], w["base_ranges"],
                                w["codes"], w["fac"], w["aid"], hq["q8"], hq["scale"], hq["k1"],
                                hq["cd"], w["route_query"], np.concatenate(
                                    [d.sample_ids for d in w["index"].dimensions]),
                                w["index"].resident_rows if resident is None else resident,
                                w["wl"].n, seg_routes, seg_off, seg_size, k, score_first)


def _explain(gi_, gd, oi, od):
    """Print the first differing (route, position) with its neighbourhood."""
    bad = np.nonzero((gi_ != oi).any(1) | (gd.view(np.uint32) != od.view(np.uint32)).any(1))[0]
    for r in bad[:3]:
        j = int(np.nonzero((gi_[r] != oi[r]) | (gd[r].view(np.uint32) != od[r].view(np.uint32)))[0][0])
        lo, hi = max(0, j - 2), j + 3
        say("route", r, "pos", j, "of", gi_.shape[1], "gpu", list(zip(gi_[r, lo:hi].tolist(), gd[r, lo:hi].tolist())),
            "oracle", list(zip(oi[r, lo:hi].tolist(), od[r, lo:hi].tolist())))


@pytest.mark.parametrize("k", [10, 200, 1000, 4096])
@pytest.mark.parametrize("segment_rows", [0, 700])
@pytest.mark.parametrize("score_first,with_pred", [(False, False), (False, True), (True, True)])
def test_range_scan_matches_oracle(gpu_ctx, rangeworld, k, segment_rows, score_first, with_pred):
    w = rangeworld
    say("range scan k", k, "segment_rows", segment_rows, "score_first", score_first,
        "pred", with_pred)
    routes = np.arange(w["routes"], dtype=np.uint32)
    pred_o = (po.PredicateArrays.from_plan(w["rs"].predicate, w["li"], base_ranges=w["base_ranges"])
              if with_pred else None)
    pred_g = w["dr"].predicate_view(w["dg"], 0.0, False) if with_pred else _lib.PredicateView()
    if segment_rows:
        plan = rp.segment_plan(routes, w["offsets"], w["sizes"], segment_rows)
        si, sd, sp = _oracle(w, pred_o, plan.route_ids, plan.offsets, plan.sizes, k, score_first)
        oi, od, op = po.merge_segments(plan.query_indptr, si, sd, sp, k)
        segs = rp.DeviceSegments(plan, merged=True)
        assert plan.count > w["routes"]
    else:
        plan = rp.segment_plan(routes, w["offsets"], w["sizes"], 1 << 30)
        oi, od, op = _oracle(w, pred_o, routes, w["offsets"], w["sizes"], k, score_first)
        segs = rp.DeviceSegments(plan, merged=False)
    ids, dists, passes = rp.rabitq_range_scan(gpu_ctx, w["rv"], w["rq"], pred_g, _routes_view(w),
                                              w["dev"]["postings"], w["index"].resident_rows, segs,
                                              k, score_first)
    torch.cuda.synchronize()
    _explain(as_u32(ids), dists.cpu().numpy(), oi, od)
    assert np.array_equal(as_u32(ids), oi)
    assert np.array_equal(dists.cpu().numpy().view(np.uint32), od.view(np.uint32))
    assert np.array_equal(as_u32(passes), op)
    assert np.all(oi[0] == U32MAX) and op[0] == 0
    assert (oi[:, 0] != U32MAX).sum() > w["routes"] // 2      # most routes find candidates


def test_posting_rows_copy(gpu_ctx, rangeworld):
    """gofann_rabitq_posting_rows: row r is the code row and {f_add,
    f_rescale, anchor} of posting sample r, zeros past the base rows."""
    w = rangeworld
    post = w["dev"]["postings"]
    rows = int(post.shape[0])
    pr = rp.PostingRows(gpu_ctx, w["rv"], post, rows)
    torch.cuda.synchronize()
    ps = post.cpu().numpy().view(np.uint32)
    ok = ps < w["wl"].n
    got_c = pr.codes.cpu().numpy()[:rows]
    got_a = pr.aux.cpu().numpy().view(np.uint32)[:rows]
    assert np.array_equal(got_c[ok], w["codes"][ps[ok]])
    assert np.array_equal(got_a[ok, 0], w["fac"][ps[ok], 0].view(np.uint32))
    assert np.array_equal(got_a[ok, 1], w["fac"][ps[ok], 1].view(np.uint32))
    assert np.array_equal(got_a[ok, 2], w["aid"][ps[ok]])
    assert not got_c[~ok].any() and not got_a[~ok].any()


@pytest.mark.parametrize("k", [200, 4096])
@pytest.mark.parametrize("segment_rows", [0, 700])
@pytest.mark.parametrize("score_first,with_pred", [(False, False), (True, True)])
def test_range_scan_resident_matches_oracle(gpu_ctx, rangeworld, k, segment_rows, score_first,
                                            with_pred):
    """The scan over posting-order copies returns the gathering scan's
    results bit for bit (the oracle's)."""
    w = rangeworld
    say("resident range scan k", k, "segment_rows", segment_rows, "score_first", score_first)
    routes = np.arange(w["routes"], dtype=np.uint32)
    pred_o = (po.PredicateArrays.from_plan(w["rs"].predicate, w["li"], base_ranges=w["base_ranges"])
              if with_pred else None)
    pred_g = w["dr"].predicate_view(w["dg"], 0.0, False) if with_pred else _lib.PredicateView()
    plan = rp.segment_plan(routes, w["offsets"], w["sizes"], segment_rows or (1 << 30))
    if segment_rows:
        si, sd, sp = _oracle(w, pred_o, plan.route_ids, plan.offsets, plan.sizes, k, score_first)
        oi, od, op = po.merge_segments(plan.query_indptr, si, sd, sp, k)
        segs = rp.DeviceSegments(plan, merged=True)
    else:
        oi, od, op = _oracle(w, pred_o, routes, w["offsets"], w["sizes"], k, score_first)
        segs = rp.DeviceSegments(plan, merged=False)
    post = w["dev"]["postings"]
    rows = rp.PostingRows(gpu_ctx, w["rv"], post, w["index"].resident_rows)
    ids, dists, passes = rp.rabitq_range_scan(gpu_ctx, w["rv"], w["rq"], pred_g, _routes_view(w),
                                              post, w["index"].resident_rows, segs, k,
                                              score_first, rows=rows)
    torch.cuda.synchronize()
    _explain(as_u32(ids), dists.cpu().numpy(), oi, od)
    assert np.array_equal(as_u32(ids), oi)
    assert np.array_equal(dists.cpu().numpy().view(np.uint32), od.view(np.uint32))
    assert np.array_equal(as_u32(passes), op)


def test_range_scan_clips_resident_rows(gpu_ctx, rangeworld):
    w = rangeworld
    say("range scan resident clip")
    k = 50
    routes = np.arange(w["routes"], dtype=np.uint32)
    resident = int(w["index"].row_count + w["index"].row_count // 3)
    plan = rp.segment_plan(routes, w["offsets"], w["sizes"], 1 << 30)
    oi, od, op = _oracle(w, None, routes, w["offsets"], w["sizes"], k, False, resident=resident)
    ids, dists, passes = rp.rabitq_range_scan(gpu_ctx, w["rv"], w["rq"], _lib.PredicateView(),
                                              _routes_view(w), w["dev"]["postings"], resident,
                                              rp.DeviceSegments(plan, merged=False), k)
    torch.cuda.synchronize()
    assert np.array_equal(as_u32(ids), oi)
    assert np.array_equal(dists.cpu().numpy().view(np.uint32), od.view(np.uint32))
    assert np.array_equal(as_u32(passes), op)


def test_range_scan_rejects_bad_shortlist(gpu_ctx, rangeworld):
    w = rangeworld
    routes = np.arange(4, dtype=np.uint32)
    plan = rp.segment_plan(routes, w["offsets"][:4], w["sizes"][:4], 1 << 30)
    segs = rp.DeviceSegments(plan, merged=False)
    for k in (0, 4097):
        rc = gpu_ctx.lib.gofann_rabitq_range_scan(
            gpu_ctx.handle, w["rv"], w["rq"], _lib.PredicateView(), _routes_view(w),
            _lib.ptr(w["dev"]["postings"]), w["index"].resident_rows, segs.view(), k, 0, None,
            None, None)
        assert rc == _lib.ERR_INVALID
