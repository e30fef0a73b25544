"""GPU parity of the RaBitQ path: query preparation against FP64 with the
reference's tolerances, the integer quantization / popcount path bit-exact
against the oracle on the same rotated input, traversal and posting scan
identical to the oracle."""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import pyoracle as po
from conftest import load_golden
from gofann_amd import _lib
from gofann_amd import index as gi
from gofann_amd import plan as gp
from gofann_amd import search as gs
from gofann_amd import synth

pytestmark = pytest.mark.gpu
U32MAX = 0xFFFFFFFF


def say(*a):
    print("[gpu-test]", *a, flush=True)
    sys.stdout.flush()


def as_u32(t):
    return t.cpu().numpy().view(np.uint32)


def prepare(ctx, queries: torch.Tensor, rotation: torch.Tensor, anchors: torch.Tensor, dim, P):
    n = queries.shape[0]
    A = anchors.shape[0]
    out = dict(rotated=torch.empty(n, P, device="cuda"), q8=torch.empty(n, P, dtype=torch.int8, device="cuda"),
               scale=torch.empty(n, device="cuda"), k1=torch.empty(n, device="cuda"),
               cd=torch.empty(n, max(A, 1), device="cuda"))
    rv = _lib.RabitqView(None, None, None, _lib.ptr(anchors), dim, P, A, 0)
    rq = _lib.RabitqQueries(_lib.ptr(out["rotated"]), _lib.ptr(out["q8"]), _lib.ptr(out["scale"]),
                            _lib.ptr(out["k1"]), _lib.ptr(out["cd"]), n)
    ctx.check(ctx.lib.gofann_rabitq_prepare_queries(ctx.handle, rv, _lib.ptr(queries), n,
                                                    _lib.ptr(rotation), rq))
    torch.cuda.synchronize()
    return out, rq


@pytest.mark.parametrize("shape", load_golden("rotation.json")["shapes"])
def test_rotation_and_centroids_vs_fp64(gpu_ctx, shape):
    """rabitq_query_rotation_test.cu:11-61 shapes and tolerances."""
    fx = load_golden("rotation.json")
    n, d, p = shape
    say("prepare", n, d, p)
    P = ((p + 63) // 64) * 64
    rng = np.random.default_rng(20260927)
    q = rng.uniform(-1, 1, (n, d)).astype(np.float32)
    r = (rng.uniform(-1, 1, (d, P)) / np.sqrt(d)).astype(np.float32)
    anchors = np.concatenate([q @ r, rng.normal(size=(5, P)).astype(np.float32)])  # rows of Y are anchors
    out, _ = prepare(gpu_ctx, torch.from_numpy(q).cuda(), torch.from_numpy(r).cuda(),
                     torch.from_numpy(anchors).cuda(), d, P)
    y = out["rotated"].cpu().numpy()
    want = q.astype(np.float64) @ r.astype(np.float64)
    a_tol, r_tol = fx["rotation_tol"]
    assert np.all(np.isfinite(y))
    assert np.all(np.abs(y - want) <= a_tol + r_tol * np.abs(want))
    cd = out["cd"].cpu().numpy()
    y64 = y.astype(np.float64)
    cw = ((y64[:, None, :] - anchors.astype(np.float64)[None]) ** 2).sum(-1)
    ca, cr = fx["centroid_tol"]
    assert np.all(cd >= 0)
    assert np.all(np.abs(cd - cw) <= ca + cr * cw)
    # integer path exact against the oracle on the GPU's rotated rows
    q8 = out["q8"].cpu().numpy()
    sc = out["scale"].cpu().numpy()
    k1 = out["k1"].cpu().numpy()
    for i in range(n):
        oq, osc, ok1 = po.rabitq_quantize(y[i])
        assert np.array_equal(q8[i], oq) and sc[i] == np.float32(osc) and k1[i] == np.float32(ok1)


def _make_rworld(degree):
    wl = synth.small_labelled(n=6000, nq=40, dim=60, k=10, sigma=0.7, labels=5, seed=31, tags=True)
    li = gi.build_label_index(wl.base, wl.label_offsets, wl.label_values, wl.num_labels,
                              wl.centroids, degree=degree, threshold=300)
    P = 128
    rot = gi.random_rotation(wl.dim, P, 31005, "cpu")
    codes, fac, aid, anchors = gi.rabitq_encode(wl.base, rot, wl.centroids)
    pl = gp.plan_queries(li, wl.query_labels)
    return wl, li, pl, rot, codes, fac, aid, anchors, P


@pytest.fixture(scope="module")
def rworld():
    return _make_rworld(32)


@pytest.fixture(scope="module")
def rworld64():
    return _make_rworld(64)


def _rviews(rw):
    wl, li, pl, rot, codes, fac, aid, anchors, P = rw
    dev = dict(codes=codes.cuda(), fac=fac.cuda(), aid=aid.cuda(), anchors=anchors.cuda(),
               rot=rot.cuda(), q=wl.queries.float().cuda())
    rv = _lib.RabitqView(_lib.ptr(dev["codes"]), _lib.ptr(dev["fac"]), _lib.ptr(dev["aid"]),
                         _lib.ptr(dev["anchors"]), wl.dim, P, anchors.shape[0], wl.n)
    return dev, rv


def _at_dim(rw, P):
    """rworld re-encoded at padded dim P (any [dim][P] matrix gives codes
    both sides score alike; a QR above 1024 would dominate the test)."""
    wl, li, pl, rot, codes, fac, aid, anchors, P0 = rw
    if P == P0:
        return rw
    if P <= 1024:
        rot = gi.random_rotation(wl.dim, P, 31005 + P, "cpu")
    else:
        rot = torch.randn(wl.dim, P, generator=torch.Generator().manual_seed(31005 + P)) / P ** 0.5
    codes, fac, aid, anchors = gi.rabitq_encode(wl.base, rot, wl.centroids)
    return wl, li, pl, rot, codes, fac, aid, anchors, P


# 128 and 1024: one candidate per lane; 2048 and 4096: whole-wave scoring
# (16-lane groups, one and two vectors per lane).
@pytest.mark.parametrize("P", [128, 1024, 2048, 4096])
def test_rabitq_score_ip_exact(gpu_ctx, rworld, P):
    rworld = _at_dim(rworld, P)
    wl, li, pl, rot, codes, fac, aid, anchors, P = rworld
    say("rabitq score P", P)
    dev, rv = _rviews(rworld)
    out, rq = prepare(gpu_ctx, dev["q"], dev["rot"], dev["anchors"], wl.dim, P)
    rng = np.random.default_rng(3)
    n = 600
    qi = np.sort(rng.integers(0, wl.queries.shape[0], n)).astype(np.uint32)
    si = rng.integers(0, wl.n, n).astype(np.uint32)
    d = torch.empty(n, device="cuda")
    ip = torch.empty(n, dtype=torch.int32, device="cuda")
    qt, st = gs.u32(qi), gs.u32(si)
    gpu_ctx.check(gpu_ctx.lib.gofann_rabitq_score(gpu_ctx.handle, rv, rq, _lib.ptr(qt), _lib.ptr(st),
                                                  n, _lib.ptr(d), _lib.ptr(ip)))
    torch.cuda.synchronize()
    q8 = out["q8"].cpu().numpy()
    sc, k1, cd = out["scale"].cpu().numpy(), out["k1"].cpu().numpy(), out["cd"].cpu().numpy()
    cn, fn, an = codes.numpy(), fac.numpy(), aid.numpy()
    L = po.lib()
    for i in range(n):
        a, b = int(qi[i]), int(si[i])
        oip = po.rabitq_ip(q8[a], cn[b], "int")
        assert int(ip[i]) == oip
        want = L.orc_rabitq_score_b1(oip, sc[a], k1[a], fn[b, 0].item(), fn[b, 1].item(), cd[a, an[b]])
        assert np.float32(d[i].item()) == np.float32(want)


# Q = 16, 40 and 96 (small and mid beams on the LDS frontier's wave-parallel
# heap operations); P = 512 is C4's 64-byte code.  At degree 32 rows scored
# a candidate per lane (P 128, 384, 512) are split between lanes l and
# l + 32: one, three (two and one) and four 16-byte vectors.
@pytest.mark.parametrize("Q", [16, 40, 96])
@pytest.mark.parametrize("P", [128, 384, 512, 2048, 4096])
@pytest.mark.parametrize("bias", [True, False])
@pytest.mark.parametrize("hash_mode,nsamp", [(_lib.PLACE_AUTO, False), (_lib.PLACE_LDS, True),
                                             (_lib.PLACE_GLOBAL, True), (_lib.PLACE_SPILL, False)])
def test_rabitq_search_matches_oracle(gpu_ctx, rworld, bias, hash_mode, nsamp, P, Q):
    _check_search(gpu_ctx, rworld, bias, hash_mode, nsamp, P, Q)


# Degree 64: every lane may hold a candidate, so rows are scored one per lane.
@pytest.mark.parametrize("P", [128, 384, 512, 4096])
@pytest.mark.parametrize("bias", [True, False])
def test_rabitq_search_degree64_matches_oracle(gpu_ctx, rworld64, bias, P):
    _check_search(gpu_ctx, rworld64, bias, _lib.PLACE_AUTO, True, P, 40)


def _check_search(gpu_ctx, rworld, bias, hash_mode, nsamp, P, Q):
    rworld = _at_dim(rworld, P)
    wl, li, pl, rot, codes, fac, aid, anchors, P = rworld
    say("rabitq search P", P, "Q", Q, "bias", bias, "hash", hash_mode, "nsamp", nsamp)
    dev, rv = _rviews(rworld)
    out, rq = prepare(gpu_ctx, dev["q"], dev["rot"], dev["anchors"], wl.dim, P)
    rs = pl.graph
    W = 30
    pred_o = po.PredicateArrays.from_plan(rs.predicate, li, alpha=0.15 if bias else 0.0,
                                          pending_base_stop=bias)
    prm_o = po.params(queue_limit=Q, result_width=W, early_stop_mode=2, bias=bias, rabitq_verdict=1)
    oi, od, ost = po.rabitq_search(li, rs, pred_o, prm_o, codes.numpy(), fac.numpy(),
                                   aid.numpy().astype(np.uint32), out["q8"].cpu().numpy(),
                                   out["scale"].cpu().numpy(), out["k1"].cpu().numpy(),
                                   out["cd"].cpu().numpy(), anchors.shape[0], P)
    dg = gs.DeviceGraph.upload(li, neighbor_samples=nsamp)
    dr = gs.DeviceRoutes.upload(rs)
    n = rs.count
    ids = torch.empty(n * W, dtype=torch.int32, device="cuda")
    dists = torch.empty(n * W, device="cuda")
    st = torch.zeros(n * 8, dtype=torch.int32, device="cuda")
    prm = gs.search_params(queue_limit=Q, result_width=W, early_stop_mode=2, bias=bias,
                           hash_mode=hash_mode)
    gpu_ctx.check(gpu_ctx.lib.gofann_rabitq_search(
        gpu_ctx.handle, rv, rq, dg.view(), dr.predicate_view(dg, 0.15 if bias else 0.0, bias),
        dr.routes_view(), prm, _lib.ptr(ids), _lib.ptr(dists), _lib.ptr(st)))
    torch.cuda.synchronize()
    assert np.array_equal(as_u32(ids).reshape(n, W), oi)
    assert np.array_equal(dists.cpu().numpy().reshape(n, W).view(np.uint32), od.view(np.uint32))
    assert np.array_equal(st.cpu().numpy().reshape(n, 8), ost)


# Padded dims 128 / 512 / 1024 take the group-per-row scan (groups of 1, 4
# and 8 lanes), 384 the thread-per-row kernel.  Forty routes are cut into
# slices and merged; reps=110 (4400 routes) runs one workgroup per route.
@pytest.mark.parametrize("P,reps,k", [(128, 1, 100), (384, 1, 100), (512, 1, 100), (1024, 1, 100),
                                      (512, 1, 10), (512, 1, 512), (512, 110, 100),
                                      (384, 110, 100)])
def test_rabitq_posting_scan_matches_oracle(gpu_ctx, rworld, P, reps, k):
    wl, li, pl, rot, codes, fac, aid, anchors, _ = _at_dim(rworld, P)
    say("rabitq posting scan P", P, "reps", reps, "k", k)
    dev, rv = _rviews((wl, li, pl, rot, codes, fac, aid, anchors, P))
    out, rq = prepare(gpu_ctx, dev["q"], dev["rot"], dev["anchors"], wl.dim, P)
    rows = [(qi, ls[0], [l for l in ls if l != ls[0]], []) for qi, ls in enumerate(wl.query_labels)]
    rows = rows * reps
    rs = gp._routeset(rows, li)
    off = np.array([li.posting_offset[r[1]] for r in rows], np.uint32)
    size = np.array([li.posting_offset[r[1] + 1] - li.posting_offset[r[1]] for r in rows], np.uint32)
    pred = po.PredicateArrays.from_plan(rs.predicate, li)
    L = po.lib()
    n = rs.count
    oi = np.empty((n, k), np.uint32)
    od = np.empty((n, k), np.float32)
    opass = np.empty(n, np.uint32)
    arrs = [np.ascontiguousarray(a) for a in (codes.numpy(), fac.numpy(), aid.numpy().astype(np.uint32),
                                               out["q8"].cpu().numpy(), out["scale"].cpu().numpy(),
                                               out["k1"].cpu().numpy(), out["cd"].cpu().numpy(),
                                               rs.route_query, li.posting_ids, off, size)]
    import ctypes as C
    assert L.orc_rabitq_posting_scan(C.byref(pred.struct), *[po.p(a) for a in arrs[:1]], C.c_uint32(P // 8),
                                     *[po.p(a) for a in arrs[1:7]], C.c_uint32(anchors.shape[0]),
                                     C.c_uint32(P), *[po.p(a) for a in arrs[7:]], C.c_uint32(n), k,
                                     po.p(oi), po.p(od), po.p(opass)) == 0
    dg = gs.DeviceGraph.upload(li)
    dr = gs.DeviceRoutes.upload(rs)
    ids = torch.empty(n * k, dtype=torch.int32, device="cuda")
    dists = torch.empty(n * k, device="cuda")
    passes = torch.empty(n, dtype=torch.int32, device="cuda")
    co, cs = gs.u32(off), gs.u32(size)
    gpu_ctx.check(gpu_ctx.lib.gofann_rabitq_posting_scan(
        gpu_ctx.handle, rv, rq, dr.predicate_view(dg, 0.0, False), _lib.ptr(dr.route_query),
        _lib.ptr(dg.posting_ids), _lib.ptr(co), _lib.ptr(cs), n, k, _lib.ptr(ids), _lib.ptr(dists),
        _lib.ptr(passes)))
    torch.cuda.synchronize()
    assert np.array_equal(as_u32(ids).reshape(n, k), oi)
    assert np.array_equal(dists.cpu().numpy().reshape(n, k).view(np.uint32), od.view(np.uint32))
    assert np.array_equal(as_u32(passes), opass)
    assert (oi[:, 0] != U32MAX).sum() > n // 2 and opass.max() > 0


@pytest.fixture(scope="module")
def cworld():
    """Label rows of 1..10 labels out of 12 (so some overflow the 7-label
    slab), one label id above 0xFFFF, and one range attribute."""
    wl = synth.small_labelled(n=7000, nq=48, dim=60, k=10, sigma=0.7, labels=4, seed=33,
                              ranges=True)
    rng = np.random.default_rng(3301)
    ids = np.array(list(range(11)) + [70000], np.uint32)
    cnt = rng.integers(1, 11, size=wl.n)
    rows = [np.sort(ids[rng.choice(12, size=int(c), replace=False)]) for c in cnt]
    wl.label_offsets = np.concatenate([[0], np.cumsum(cnt)]).astype(np.uint32)
    wl.label_values = np.concatenate(rows).astype(np.uint32)
    wl.num_labels = 70001
    li = gi.build_label_index(wl.base, wl.label_offsets, wl.label_values, wl.num_labels,
                              wl.centroids, degree=32, threshold=10**9)
    P = 128
    rot = gi.random_rotation(wl.dim, P, 33005, "cpu")
    codes, fac, aid, anchors = gi.rabitq_encode(wl.base, rot, wl.centroids)
    # routes: anchor label, 0..2 residual labels, the query's range on half
    routes = []
    for rep in range(3):
        for qi in range(wl.queries.shape[0]):
            lab = [int(x) for x in rng.choice(ids, size=int(rng.integers(1, 4)), replace=False)]
            rngs = wl.query_ranges[qi] if (qi + rep) % 2 == 0 else []
            routes.append((qi, lab[0], lab[1:], rngs))
    return wl, li, routes, rot, codes, fac, aid, anchors, P


# target_rows 97 cuts every posting into many segments; 1 << 20 keeps one
# segment per route.  Each column set (none, codes, predicate columns,
# both) must give the oracle's results bit for bit.
@pytest.mark.parametrize("target", [97, 1 << 20])
@pytest.mark.parametrize("codes_cols,pred_cols", [(False, False), (True, False), (False, True),
                                                  (True, True)])
def test_rabitq_posting_scan_segments_matches_oracle(gpu_ctx, cworld, target, codes_cols,
                                                     pred_cols):
    from gofann_amd import range_posting as rp
    wl, li, routes, rot, codes, fac, aid, anchors, P = cworld
    k = 40
    say("posting scan segments target", target, "codes", codes_cols, "pred", pred_cols)
    dev, rv = _rviews((wl, li, None, rot, codes, fac, aid, anchors, P))
    out, rq = prepare(gpu_ctx, dev["q"], dev["rot"], dev["anchors"], wl.dim, P)
    rs = gp._routeset(routes, li)
    n = rs.count
    off = np.array([li.posting_offset[r[1]] for r in routes], np.uint32)
    size = np.array([li.posting_offset[r[1] + 1] - li.posting_offset[r[1]] for r in routes],
                    np.uint32)
    pred = po.PredicateArrays.from_plan(rs.predicate, li, base_ranges=wl.base_ranges)
    oi, od, opass = po.posting_scan_rabitq(
        pred, codes.numpy(), fac.numpy(), aid.numpy().astype(np.uint32),
        out["q8"].cpu().numpy(), out["scale"].cpu().numpy(), out["k1"].cpu().numpy(),
        out["cd"].cpu().numpy(), rs.route_query, li.posting_ids, off, size, k)
    dg = gs.DeviceGraph.upload(li)
    dr = gs.DeviceRoutes.upload(rs, wl.base_ranges)
    pv = dr.predicate_view(dg, 0.0, False)
    total = int(li.posting_offset[-1])
    plan = rp.segment_plan(np.arange(n), off.astype(np.uint64), size.astype(np.uint64), target)
    assert target > 1000 or plan.count > 4 * n
    segs = rp.DeviceSegments(plan)
    rows = rp.PostingRows(gpu_ctx, rv, dg.posting_ids, total) if codes_cols else None
    cols = rp.PostingPredicateColumns(gpu_ctx, pv, dg.posting_ids, total) if pred_cols else None
    ids, dists, passes = rp.rabitq_posting_scan_segments(
        gpu_ctx, rv, rq, pv, dr.route_query, dg.posting_ids, total, segs, k, rows=rows, cols=cols)
    torch.cuda.synchronize()
    assert np.array_equal(as_u32(ids).reshape(n, k), oi)
    assert np.array_equal(dists.cpu().numpy().reshape(n, k).view(np.uint32), od.view(np.uint32))
    assert np.array_equal(as_u32(passes), opass)
    assert (oi[:, 0] != U32MAX).sum() > n // 2 and opass.max() > 0
    if cols is not None:
        # the slab of a row with more than 7 labels, or with label 70000,
        # is the overflow form; the others hold the row's labels
        slab = cols.slab.cpu().numpy().view(np.uint32)
        pid = li.posting_ids
        lo, lv = wl.label_offsets, wl.label_values
        for r in range(0, total, 97):
            s = int(pid[r])
            labs = lv[lo[s]:lo[s + 1]]
            cnt = slab[r, 0] & 0xFFFF
            if len(labs) > 7 or labs.max() > 0xFFFF:
                assert cnt == 0xFFFF
            else:
                got = [(slab[r, (h >> 1)] >> (16 * (h & 1))) & 0xFFFF for h in range(1, cnt + 1)]
                assert cnt == len(labs) and got == labs.tolist()
            assert cols.ranges[r].item() == wl.base_ranges[s, 0]


_SHARE_CODES = {}


def _uncapped_share_plan(rp, plan):
    """Every plan segment of one (offset, size) in a single item, however
    many: items above 16 routes take the kernel's extra passes."""
    order = np.lexsort((np.arange(plan.count), plan.sizes, plan.offsets))
    o, sz = plan.offsets[order], plan.sizes[order]
    new = np.r_[True, (o[1:] != o[:-1]) | (sz[1:] != sz[:-1])]
    starts = np.flatnonzero(new)
    begin = np.r_[starts, plan.count].astype(np.uint32)
    return rp.SharePlan(o[starts].astype(np.uint64), sz[starts].astype(np.uint64), begin,
                        order.astype(np.uint32))


def _shared_scan_case(gpu_ctx, cworld, P, target, k, per_item, repeat=1):
    from gofann_amd import range_posting as rp
    wl, li, routes, _rot, _codes, _fac, _aid, _anchors, _P = cworld
    routes = list(routes) * repeat
    say("posting scan shared P", P, "target", target, "k", k, "per_item", per_item,
        "routes", len(routes))
    if P not in _SHARE_CODES:
        rot = gi.random_rotation(wl.dim, P, 33005 + P, "cpu")
        _SHARE_CODES[P] = (rot,) + tuple(gi.rabitq_encode(wl.base, rot, wl.centroids))
    rot, codes, fac, aid, anchors = _SHARE_CODES[P]
    dev, rv = _rviews((wl, li, None, rot, codes, fac, aid, anchors, P))
    out, rq = prepare(gpu_ctx, dev["q"], dev["rot"], dev["anchors"], wl.dim, P)
    rs = gp._routeset(routes, li)
    n = rs.count
    off = np.array([li.posting_offset[r[1]] for r in routes], np.uint32)
    size = np.array([li.posting_offset[r[1] + 1] - li.posting_offset[r[1]] for r in routes],
                    np.uint32)
    pred = po.PredicateArrays.from_plan(rs.predicate, li, base_ranges=wl.base_ranges)
    oi, od, opass = po.posting_scan_rabitq(
        pred, codes.numpy(), fac.numpy(), aid.numpy().astype(np.uint32),
        out["q8"].cpu().numpy(), out["scale"].cpu().numpy(), out["k1"].cpu().numpy(),
        out["cd"].cpu().numpy(), rs.route_query, li.posting_ids, off, size, k)
    dg = gs.DeviceGraph.upload(li)
    dr = gs.DeviceRoutes.upload(rs, wl.base_ranges)
    pv = dr.predicate_view(dg, 0.0, False)
    total = int(li.posting_offset[-1])
    plan = rp.segment_plan(np.arange(n), off.astype(np.uint64), size.astype(np.uint64), target)
    segs = rp.DeviceSegments(plan)
    sp = rp.share_plan(plan, per_item) if per_item else _uncapped_share_plan(rp, plan)
    counts = np.diff(sp.begin.astype(np.int64))
    assert sp.items < plan.count  # segments of one label share items
    if per_item:
        assert counts.max() <= per_item
    else:
        assert counts.max() > 2 * rp.SHARE_ROUTES  # three passes over some items
    share = rp.DeviceShare(sp)
    rows = rp.PostingRows(gpu_ctx, rv, dg.posting_ids, total)
    cols = rp.PostingPredicateColumns(gpu_ctx, pv, dg.posting_ids, total)
    ids, dists, passes = rp.rabitq_posting_scan_segments(
        gpu_ctx, rv, rq, pv, dr.route_query, dg.posting_ids, total, segs, k, rows=rows,
        cols=cols, share=share)
    torch.cuda.synchronize()
    assert np.array_equal(as_u32(ids).reshape(n, k), oi)
    assert np.array_equal(dists.cpu().numpy().reshape(n, k).view(np.uint32), od.view(np.uint32))
    assert np.array_equal(as_u32(passes), opass)
    assert (oi[:, 0] != U32MAX).sum() > n // 2 and opass.max() > 0


# The label-shared scan (one workgroup per label segment, a wave per route):
# P 128 to 1024 (one to eight code vectors per row; 1024 is the largest LDS
# layout, 32 plane words per route), segments cut small, across tile
# boundaries (700 rows) and whole; shortlists of 40 and 100.
@pytest.mark.parametrize("P", [128, 256, 512, 1024])
@pytest.mark.parametrize("target", [97, 700, 1 << 20])
@pytest.mark.parametrize("k", [40, 100])
def test_rabitq_posting_scan_shared_matches_oracle(gpu_ctx, cworld, P, target, k):
    _shared_scan_case(gpu_ctx, cworld, P, target, k, 16)


# Items of fewer than 16 routes (5 per item), and items of more than 32
# routes (every route of a label segment in one item; the route set is
# repeated three times), which the kernel serves in passes of 16 slots.
@pytest.mark.parametrize("P", [256, 1024])
@pytest.mark.parametrize("per_item", [5, 0])
def test_rabitq_posting_scan_shared_item_sizes(gpu_ctx, cworld, P, per_item):
    _shared_scan_case(gpu_ctx, cworld, P, 700, 40, per_item, repeat=1 if per_item else 3)


def test_streamed_host_rerank_matches_direct(gpu_ctx, rworld):
    """RaBitQ traversal in route chunks with each chunk's shortlist streamed
    to the host rerank pool (search.StreamedRerank): the chunked shortlists
    equal one unchunked launch, and the streamed rerank equals the pool's
    direct rerank of the same shortlists, bit for bit."""
    wl, li, pl, rot, codes, fac, aid, anchors, P = rworld
    say("streamed host rerank")
    dev, rv = _rviews(rworld)
    out, rq = prepare(gpu_ctx, dev["q"], dev["rot"], dev["anchors"], wl.dim, P)
    rs = pl.graph
    n, W = rs.count, 30
    dg = gs.DeviceGraph.upload(li)
    dr = gs.DeviceRoutes.upload(rs)
    pv = dr.predicate_view(dg, 0.15, True)
    prm = gs.search_params(queue_limit=40, result_width=W, early_stop_mode=2, bias=True)

    def launch(ids, dists, c0, c1):
        gpu_ctx.check(gpu_ctx.lib.gofann_rabitq_search(
            gpu_ctx.handle, rv, rq, dg.view(), pv, dr.routes_view(c0, c1), prm, _lib.ptr(ids),
            _lib.ptr(dists), None))

    ids_a = torch.empty(n * W, dtype=torch.int32, device="cuda")
    d_a = torch.empty(n * W, device="cuda")
    launch(ids_a, d_a, 0, n)
    torch.cuda.synchronize()
    sl = as_u32(ids_a).reshape(n, W)
    hr = gs.HostRerank(wl.base.numpy(), wl.queries.numpy(), threads=4)
    want_i, want_d = hr.rerank(sl, rs.route_query, 10)
    ids_b = torch.full((n * W,), -1, dtype=torch.int32, device="cuda")
    d_b = torch.empty(n * W, device="cuda")
    sr = gs.StreamedRerank(hr, n, W)
    tasks = [(c0, min(n, c0 + 7), (lambda c0=c0: launch(ids_b, d_b, c0, min(n, c0 + 7))))
             for c0 in range(0, n, 7)]
    got_i = np.empty((n, 10), np.uint32)
    got_d = np.empty((n, 10), np.float32)
    sr.run(tasks, ids_b, rs.route_query, 10, got_i, got_d)
    torch.cuda.synchronize()
    assert np.array_equal(as_u32(ids_b).reshape(n, W), sl)
    assert np.array_equal(got_i, want_i)
    assert np.array_equal(got_d.view(np.uint32), want_d.view(np.uint32))
    assert sr.timing["gpu_ms"] > 0 and sr.timing["wall_ms"] >= sr.timing["gpu_ms"] * 0.5
    assert (want_i[:, 0] != U32MAX).sum() > n // 2
    hr.close()


@pytest.mark.parametrize("Q,W", [(80, 30), (200, 100), (448, 100)])
@pytest.mark.parametrize("hash_mode", [_lib.PLACE_LDS, _lib.PLACE_GLOBAL])
@pytest.mark.parametrize("bias", [True, False])
def test_rabitq_pair_kernel_matches_oracle(gpu_ctx, rworld, Q, W, hash_mode, bias, monkeypatch):
    """Two routes per wave (degree 32, LDS frontier, rabitq_pair.hip, asked
    for by GOFANN_RABITQ_PAIR=1) on an odd number of routes, so the last wave
    runs one, and the one-route kernel with its wave-parallel frontier (Q + 2
    up to 512 slots, so pop_max follows pairs past 64): ids, distance bits
    and counters identical to the oracle in both."""
    wl, li, pl, rot, codes, fac, aid, anchors, P = _at_dim(rworld, 512)
    say("rabitq pair kernel Q", Q, "W", W, "hash", hash_mode, "bias", bias)
    dev, rv = _rviews((wl, li, pl, rot, codes, fac, aid, anchors, P))
    out, rq = prepare(gpu_ctx, dev["q"], dev["rot"], dev["anchors"], wl.dim, P)
    rs = pl.graph
    n = rs.count if rs.count % 2 else rs.count - 1
    pred_o = po.PredicateArrays.from_plan(rs.predicate, li, alpha=0.15 if bias else 0.0,
                                          pending_base_stop=bias)
    prm_o = po.params(queue_limit=Q, result_width=W, early_stop_mode=2, bias=bias,
                      rabitq_verdict=1)
    oi, od, ost = po.rabitq_search(li, rs, pred_o, prm_o, codes.numpy(), fac.numpy(),
                                   aid.numpy().astype(np.uint32), out["q8"].cpu().numpy(),
                                   out["scale"].cpu().numpy(), out["k1"].cpu().numpy(),
                                   out["cd"].cpu().numpy(), anchors.shape[0], P)
    dg = gs.DeviceGraph.upload(li, neighbor_samples=True)
    dr = gs.DeviceRoutes.upload(rs)
    prm = gs.search_params(queue_limit=Q, result_width=W, early_stop_mode=2, bias=bias,
                           hash_mode=hash_mode)

    def run():
        ids = torch.full((rs.count * W,), -7, dtype=torch.int32, device="cuda")
        dists = torch.empty(rs.count * W, device="cuda")
        st = torch.zeros(rs.count * 8, dtype=torch.int32, device="cuda")
        gpu_ctx.check(gpu_ctx.lib.gofann_rabitq_search(
            gpu_ctx.handle, rv, rq, dg.view(), dr.predicate_view(dg, 0.15 if bias else 0.0, bias),
            dr.routes_view(0, n), prm, _lib.ptr(ids), _lib.ptr(dists), _lib.ptr(st)))
        torch.cuda.synchronize()
        return (as_u32(ids).reshape(rs.count, W), dists.cpu().numpy().reshape(rs.count, W),
                st.cpu().numpy().reshape(rs.count, 8))

    for pair in ("1", "0"):
        monkeypatch.setenv("GOFANN_RABITQ_PAIR", pair)
        gi_, gd, gst = run()
        assert np.array_equal(gi_[:n], oi[:n]), pair
        assert np.array_equal(gd[:n].view(np.uint32), od[:n].view(np.uint32)), pair
        assert np.array_equal(gst[:n], ost[:n]), pair
        assert np.all(gi_[n:] == np.uint32(0xFFFFFFF9))  # routes outside the launch untouched
    assert (oi[:n, 0] != U32MAX).sum() > n // 2
    if Q > 300:  # some frontier grew past 260 slots: pairs 64.. have children
        assert ost[:n, 6].max() > 300


@pytest.fixture(scope="module")
def rrange_world():
    """Tags and one numeric attribute: route predicates with label and
    range atoms, for per-sample records that carry both."""
    wl = synth.small_labelled(n=6000, nq=40, dim=60, k=10, sigma=0.7, labels=5, seed=37, tags=True,
                              ranges=True)
    li = gi.build_label_index(wl.base, wl.label_offsets, wl.label_values, wl.num_labels,
                              wl.centroids, degree=32, threshold=300)
    pl = gp.plan_queries(li, wl.query_labels, wl.query_ranges)
    return wl, li, pl


@pytest.mark.parametrize("P", [128, 512, 4096])
@pytest.mark.parametrize("bias", [True, False])
@pytest.mark.parametrize("hash_mode,Q", [(_lib.PLACE_AUTO, 40), (_lib.PLACE_GLOBAL, 96),
                                         (_lib.PLACE_LDS, 300)])
@pytest.mark.parametrize("overflow", [0, 3])
def test_rabitq_search_with_records_matches_oracle(gpu_ctx, rrange_world, P, bias, hash_mode, Q,
                                                   overflow, monkeypatch):
    """The traversal reading per-sample records (code row, f_add, f_rescale,
    anchor id, attribute value, label slab in one line) in place of the
    separate arrays, its predicate reading the slab and the attribute from
    the same records: ids, distance bits and counters identical to the
    oracle, in the one-route and the two-routes-per-wave kernels; overflow 3
    forces every third row's labels through the CSR."""
    wl, li, pl = rrange_world
    if P <= 1024:
        rot = gi.random_rotation(wl.dim, P, 37005 + P, "cpu")
    else:
        rot = torch.randn(wl.dim, P, generator=torch.Generator().manual_seed(37005 + P)) / P ** 0.5
    codes, fac, aid, anchors = gi.rabitq_encode(wl.base, rot, wl.centroids)
    say("rabitq records P", P, "bias", bias, "hash", hash_mode, "Q", Q, "overflow", overflow)
    rw = (wl, li, pl, rot, codes, fac, aid, anchors, P)
    dev, rv = _rviews(rw)
    out, rq = prepare(gpu_ctx, dev["q"], dev["rot"], dev["anchors"], wl.dim, P)
    rs = pl.graph
    W = 30
    pred_o = po.PredicateArrays.from_plan(rs.predicate, li, wl.base_ranges,
                                          alpha=0.15 if bias else 0.0, pending_base_stop=bias)
    prm_o = po.params(queue_limit=Q, result_width=W, early_stop_mode=2, bias=bias, rabitq_verdict=1)
    oi, od, ost = po.rabitq_search(li, rs, pred_o, prm_o, codes.numpy(), fac.numpy(),
                                   aid.numpy().astype(np.uint32), out["q8"].cpu().numpy(),
                                   out["scale"].cpu().numpy(), out["k1"].cpu().numpy(),
                                   out["cd"].cpu().numpy(), anchors.shape[0], P)
    rec = gs.RabitqRecords.build(dev["codes"], dev["fac"], dev["aid"], wl.base_ranges,
                                 li.csr_offsets, li.csr_labels, chunk=2500,
                                 overflow_every=overflow)
    assert rec.stride % 128 == 0 and rec.stride >= P // 8 + 12 + 4 + 16
    rv.records, rv.record_stride = rec.view_fields()
    dg = gs.DeviceGraph.upload(li, neighbor_samples=True)
    dr = gs.DeviceRoutes.upload(rs, wl.base_ranges)
    pv = dr.predicate_view(dg, 0.15 if bias else 0.0, bias, records=rec)
    assert pv.range_columns == 1 and pv.range_stride == rec.stride // 4
    prm = gs.search_params(queue_limit=Q, result_width=W, early_stop_mode=2, bias=bias,
                           hash_mode=hash_mode)
    n = rs.count
    for pair in ("0", "1"):
        monkeypatch.setenv("GOFANN_RABITQ_PAIR", pair)
        ids = torch.empty(n * W, dtype=torch.int32, device="cuda")
        dists = torch.empty(n * W, device="cuda")
        st = torch.zeros(n * 8, dtype=torch.int32, device="cuda")
        gpu_ctx.check(gpu_ctx.lib.gofann_rabitq_search(
            gpu_ctx.handle, rv, rq, dg.view(), pv, dr.routes_view(), prm, _lib.ptr(ids),
            _lib.ptr(dists), _lib.ptr(st)))
        torch.cuda.synchronize()
        assert np.array_equal(as_u32(ids).reshape(n, W), oi), pair
        assert np.array_equal(dists.cpu().numpy().reshape(n, W).view(np.uint32),
                              od.view(np.uint32)), pair
        assert np.array_equal(st.cpu().numpy().reshape(n, 8), ost), pair
    assert (oi[:, 0] != U32MAX).sum() > n // 3


def test_rabitq_records_layout(gpu_ctx):
    """Record bytes: code row at 0, f_add and f_rescale, anchor id, the
    attribute columns, the 16-byte label slab at a 16-byte offset, stride a
    multiple of 128."""
    n, cb = 50, 64
    g = torch.Generator().manual_seed(5)
    codes = torch.randint(0, 256, (n, cb), generator=g, dtype=torch.uint8)
    fac = torch.randn(n, 3, generator=g)
    aid = torch.randint(0, 1000, (n,), generator=g, dtype=torch.int32)
    br = torch.randn(n, 2, generator=g).numpy()
    off = np.arange(0, 2 * n + 1, 2, dtype=np.uint32)
    lab = np.tile(np.array([3, 9], np.uint32), n)
    rec = gs.RabitqRecords.build(codes.cuda(), fac.cuda(), aid.cuda(), br, off, lab, chunk=7)
    d = rec.data.cpu().numpy()
    assert rec.stride == 128 and rec.range_offset == 76 and rec.slab_offset == 96
    assert np.array_equal(d[:, :cb], codes.numpy())
    assert np.array_equal(d[:, cb:cb + 8].copy().view(np.float32), fac[:, :2].numpy())
    assert np.array_equal(d[:, cb + 8:cb + 12].copy().view(np.int32)[:, 0], aid.numpy())
    assert np.array_equal(d[:, 76:84].copy().view(np.float32), br)
    sl = d[:, 96:112].copy().view(np.uint16)
    assert np.all(sl[:, 0] == 2) and np.all(sl[:, 1] == 3) and np.all(sl[:, 2] == 9)
