"""GPU parity of the full-GPU exact route (gofann_exact_search): ids,
distance bits and the eight per-route counters identical to the oracle,
across visited-set placements, neighbour-sample tables, early-stop modes,
beam sizes, route predicates and legacy bit/range filters, and every
distance path (u8 rows of fixed length 128/192/256, dim % 16 == 0, dim % 4
== 0, any dim; f32 and f16 rows in the warp order); and the exact posting
scans in both summation orders."""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import pyoracle as po
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


def _world(dim, seed, n=5000, nq=40):
    wl = synth.small_labelled(n=n, nq=nq, dim=dim, k=10, sigma=0.7, labels=5, seed=seed, tags=True,
                              dtype="u8")
    li = gi.build_label_index(wl.base, wl.label_offsets, wl.label_values, wl.num_labels,
                              wl.centroids, degree=32, threshold=300)
    pl = gp.plan_queries(li, wl.query_labels)
    return wl, li, pl.graph


@pytest.fixture(scope="module")
def eworld(gpu_ctx):
    return _world(128, 51)


ELEM = {np.dtype(np.uint8): _lib.ELEM_U8, np.dtype(np.float32): _lib.ELEM_F32,
        np.dtype(np.float16): _lib.ELEM_F16}


def _run(ctx, wl, li, rs, pred_o, pred_g, Q, topk, mode, hash_mode, nsamp, max_steps=0,
         finish=1, legacy=None, rows=None):
    base, q = rows if rows is not None else (wl.base.numpy(), wl.queries.numpy())
    kw = {}
    if legacy is not None:
        kw = dict(row_filter_mask=legacy["rmask"], query_filter_bits=legacy["qbits"],
                  range_modes=legacy["modes"], range_lower=legacy["lo"], range_upper=legacy["hi"],
                  base_range_values=legacy["brv"])
    oi, od, ost = po.exact_search(li, rs, pred_o, base, q, queue_limit=Q, topk=topk,
                                  early_stop_mode=mode, finish_limit=finish, max_steps=max_steps,
                                  label_size=li.label_size, **kw)
    dg = gs.DeviceGraph.upload(li, neighbor_samples=nsamp)
    dr = gs.DeviceRoutes.upload(rs)
    dev = dict(base=torch.from_numpy(np.ascontiguousarray(base)).cuda(),
               q=torch.from_numpy(np.ascontiguousarray(q)).cuda(), ls=gs.u32(li.label_size))
    rv = dr.routes_view()
    if legacy is not None:
        for k in ("rmask", "qbits"):
            dev[k] = torch.from_numpy(legacy[k].view(np.int64)).cuda()
        dev["modes"] = torch.from_numpy(legacy["modes"]).cuda()
        dev["lo"] = torch.from_numpy(legacy["lo"]).cuda()
        dev["hi"] = torch.from_numpy(legacy["hi"]).cuda()
        dev["brv"] = torch.from_numpy(legacy["brv"]).cuda()
        rv.row_filter_mask, rv.query_filter_bits = _lib.ptr(dev["rmask"]), _lib.ptr(dev["qbits"])
        rv.range_modes, rv.range_lower = _lib.ptr(dev["modes"]), _lib.ptr(dev["lo"])
        rv.range_upper, rv.base_range_values = _lib.ptr(dev["hi"]), _lib.ptr(dev["brv"])
        rv.range_count = legacy["modes"].shape[1]
    n = rs.count
    ids = torch.empty(n * topk, dtype=torch.int32, device="cuda")
    dists = torch.empty(n * topk, device="cuda")
    st = torch.zeros(n * 8, dtype=torch.int32, device="cuda")
    prm = _lib.ExactParams(Q, finish, mode, max_steps, topk, hash_mode)
    ctx.check(ctx.lib.gofann_exact_search(ctx.handle, _lib.ptr(dev["base"]), ELEM[base.dtype], wl.dim,
                                          wl.n, _lib.ptr(dev["q"]), dg.view(), _lib.ptr(dev["ls"]),
                                          pred_g(dr, dg), rv, prm, _lib.ptr(ids), _lib.ptr(dists),
                                          _lib.ptr(st)))
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy().view(np.uint32).reshape(n, topk), oi)
    assert np.array_equal(dists.cpu().numpy().reshape(n, topk).view(np.uint32), od.view(np.uint32))
    assert np.array_equal(st.cpu().numpy().reshape(n, 8), ost)
    return oi, ost


PLACE = {"auto": (_lib.PLACE_AUTO, False), "lds-nsamp": (_lib.PLACE_LDS, True),
         "global": (_lib.PLACE_GLOBAL, False), "spill-nsamp": (_lib.PLACE_SPILL, True)}


@pytest.mark.parametrize("place", list(PLACE))
# Beams up to 510 admit through the wave-parallel heap operations on the
# LDS frontier; past 512 slots (Q = 600) admission takes the serial lane-0
# sifts.
@pytest.mark.parametrize("mode,Q", [(2, 32), (0, 62), (2, 64), (2, 80), (1, 128), (2, 300),
                                    (2, 600)])
@pytest.mark.parametrize("with_pred", [False, True])
def test_exact_search_matches_oracle(gpu_ctx, eworld, place, mode, Q, with_pred):
    wl, li, rs = eworld
    hash_mode, nsamp = PLACE[place]
    say("exact search", place, "mode", mode, "Q", Q, "pred", with_pred)
    pred_o = po.PredicateArrays.from_plan(rs.predicate, li) if with_pred else None

    def pred_g(dr, dg):
        return dr.predicate_view(dg, 0.0, False) if with_pred else _lib.PredicateView()

    oi, ost = _run(gpu_ctx, wl, li, rs, pred_o, pred_g, Q, 10, mode, hash_mode, nsamp,
                   max_steps=300 if mode == 1 else 0, finish=2)
    assert (oi[:, 0] != U32MAX).sum() > rs.count // 2
    assert ost[:, 0].max() > 5


@pytest.fixture(scope="module")
def c2_shape_world(gpu_ctx):
    """The C2 bench shape: dim 192 u8 (fixed 12-chunk rows), degree 64, tags,
    trained k-means buckets, medoid seeds."""
    wl = synth.small_labelled(n=9000, nq=48, dim=192, k=14, sigma=0.7, labels=6, seed=57,
                              tags=True, dtype="u8")
    cen = gi.train_kmeans(wl.base, 14, seed=57)
    li = gi.build_label_index(wl.base, wl.label_offsets, wl.label_values, wl.num_labels, cen,
                              degree=64, threshold=300)
    return wl, li, gp.plan_queries(li, wl.query_labels).graph


@pytest.mark.parametrize("place", list(PLACE))
@pytest.mark.parametrize("mode,Q", [(2, 32), (2, 62), (2, 96), (2, 126), (0, 128), (2, 300)])
def test_exact_search_degree64_c2_shape(gpu_ctx, c2_shape_world, place, mode, Q):
    """Degree 64: lanes 32..63 of load_node/keep, the 64-bit ballot
    compaction and admissions of more than 32 neighbours per step."""
    wl, li, rs = c2_shape_world
    hash_mode, nsamp = PLACE[place]
    say("exact search degree 64", place, "mode", mode, "Q", Q)
    pred_o = po.PredicateArrays.from_plan(rs.predicate, li)
    oi, ost = _run(gpu_ctx, wl, li, rs, pred_o, lambda dr, dg: dr.predicate_view(dg, 0.0, False),
                   Q, 10, mode, hash_mode, nsamp, finish=2)
    assert (li.graph[:, 32:] != U32MAX).any(1).mean() > 0.5
    assert ost[:, 6].max() > 32  # some step admitted more than 32 neighbours overall
    if Q > 260:  # some frontier grew past 260 slots: pairs 64.. have children
        assert ost[:, 6].max() > 300
    assert (oi[:, 0] != U32MAX).sum() > rs.count // 2


def test_exact_search_legacy_filters_and_topk1(gpu_ctx, eworld):
    wl, li, rs = eworld
    say("exact search legacy filters")
    rng = np.random.default_rng(9)
    rc = 2
    legacy = dict(rmask=rng.integers(1, 4, li.row_to_sample.shape[0]).astype(np.uint64),
                  qbits=rng.integers(1, 4, rs.count).astype(np.uint64),
                  modes=rng.integers(0, 4, (rs.count, rc)).astype(np.uint8),
                  brv=rng.integers(0, 20, (wl.n, rc)).astype(np.float32))
    legacy["lo"] = rng.integers(0, 8, (rs.count, rc)).astype(np.float32)
    legacy["hi"] = legacy["lo"] + rng.integers(4, 12, (rs.count, rc)).astype(np.float32)
    for topk in (1, 10):
        _run(gpu_ctx, wl, li, rs, None, lambda dr, dg: _lib.PredicateView(), 48, topk, 2,
             _lib.PLACE_AUTO, True, legacy=legacy)


@pytest.mark.parametrize("dim", [44, 45, 48, 192, 256])
def test_exact_search_distance_paths(gpu_ctx, dim):
    wl, li, rs = _world(dim, 60 + dim, n=3000, nq=24)
    say("exact search dim", dim)
    _run(gpu_ctx, wl, li, rs, None, lambda dr, dg: _lib.PredicateView(), 32, 10, 2,
         _lib.PLACE_AUTO, False)


@pytest.mark.parametrize("overflow", [0, 3])
def test_exact_search_label_slab(gpu_ctx, eworld, overflow):
    """The route predicate reading each node's labels from a 16-byte slab in
    per-sample records (fetched with the adjacency row at pickup) in place
    of the CSR: results identical to the oracle's; overflow 3 sends every
    third row through the CSR."""
    wl, li, rs = eworld
    say("exact search label slab overflow", overflow)
    rec = gs.SampleRecords.build(torch.zeros(wl.n, 16, dtype=torch.uint8), li.csr_offsets,
                                 li.csr_labels, overflow_every=overflow)
    pred_o = po.PredicateArrays.from_plan(rs.predicate, li)
    for place, mode, Q in (("auto", 2, 48), ("spill-nsamp", 2, 96)):
        hash_mode, nsamp = PLACE[place]
        _run(gpu_ctx, wl, li, rs, pred_o,
             lambda dr, dg: dr.predicate_view(dg, 0.0, False, records=rec), Q, 10, mode,
             hash_mode, nsamp, finish=2)


def _float_world(dim, seed, n=4000, nq=32):
    wl = synth.small_labelled(n=n, nq=nq, dim=dim, k=10, sigma=0.7, labels=5, seed=seed,
                              tags=True)
    li = gi.build_label_index(wl.base, wl.label_offsets, wl.label_values, wl.num_labels,
                              wl.centroids, degree=32, threshold=300)
    return wl, li, gp.plan_queries(li, wl.query_labels).graph


@pytest.mark.parametrize("dim", [37, 100, 128, 512, 1031, 2049, 4096])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_exact_search_float_rows(gpu_ctx, dim, dtype):
    """f32 and f16 rows (and queries of the same type): distances in the
    reference's warp order, bit-identical to the oracle, with every
    visited-set placement; odd dim takes the per-element f16 path, 100
    leaves partials of unequal length.  Rows over 4 KB (f32 1031 and up,
    f16 2049 and up; 4096 is C3's shape) take the long-row kernel, whose
    lanes load 32 row words at a time: 1031 and 2049 leave a tail shorter
    than one such batch."""
    wl, li, rs = _float_world(dim, 70 + dim)
    t = np.float16 if dtype == "f16" else np.float32
    rows = (wl.base.numpy().astype(t), wl.queries.numpy().astype(t))
    pred_o = po.PredicateArrays.from_plan(rs.predicate, li)
    for place, mode, Q, with_pred in (("auto", 2, 32, False), ("lds-nsamp", 2, 80, True),
                                      ("global", 0, 128, False), ("spill-nsamp", 2, 300, True)):
        hash_mode, nsamp = PLACE[place]
        say("exact search float rows", dtype, "dim", dim, place, "Q", Q, "pred", with_pred)

        def pred_g(dr, dg):
            return dr.predicate_view(dg, 0.0, False) if with_pred else _lib.PredicateView()

        oi, ost = _run(gpu_ctx, wl, li, rs, pred_o if with_pred else None, pred_g, Q, 10, mode,
                       hash_mode, nsamp, finish=2, rows=rows)
        assert (oi[:, 0] != U32MAX).sum() > rs.count // 2
        assert ost[:, 0].max() > 5


@pytest.fixture(scope="module")
def scan_worlds(gpu_ctx):
    out = {}
    for dim in (37, 128, 512, 4096):
        wl = synth.small_labelled(n=6000, nq=24, dim=dim, k=10, sigma=0.7, labels=5,
                                  seed=90 + dim, tags=True)
        li = gi.build_label_index(wl.base, wl.label_offsets, wl.label_values, wl.num_labels,
                                  wl.centroids, degree=16, threshold=300)
        out[dim] = (wl, li)
    return out


def _scan_lists(rng, n, routes):
    """Posting lists with duplicates, UINT32_MAX, ids past the base, an
    empty list and lists longer than one LDS chunk."""
    sizes = rng.integers(0, 700, routes).astype(np.uint32)
    sizes[0] = 0
    sizes[1] = 5000
    sizes[2] = 2048
    offs = np.zeros(routes, np.uint32)
    offs[1:] = np.cumsum(sizes)[:-1]
    ids = rng.integers(0, n, int(sizes.sum())).astype(np.uint32)
    ids[offs[1] + 3000: offs[1] + 3100] = ids[offs[1]: offs[1] + 100]
    ids[rng.integers(0, len(ids), len(ids) // 20)] = U32MAX
    ids[rng.integers(0, len(ids), len(ids) // 20)] = n + 3
    return ids, offs, sizes


@pytest.mark.parametrize("dim", [37, 128, 512, 4096])
@pytest.mark.parametrize("dtype", ["u8", "f32", "f16"])
@pytest.mark.parametrize("order", [_lib.EXACT_ORDER_SERIAL, _lib.EXACT_ORDER_WARP])
def test_exact_posting_scan_matches_oracle(gpu_ctx, scan_worlds, dim, dtype, order):
    """gofann_exact_posting_scan: ids, distance bits and pass counts equal
    the oracle's in both summation orders, with and without the route
    predicate, for topk 1, 10 and 64.  Row lengths cover the serial order's
    LDS tiles (rows of 16-byte multiples, 4096 at the C3 shape) and its
    thread-per-row path (dim 37), and the warp order's unaligned blocks."""
    wl, li = scan_worlds[dim]
    x, qx = wl.base.numpy(), wl.queries.numpy()
    if dtype == "u8":
        lo, hi = float(x.min()), float(x.max())
        base = np.clip(np.round((x - lo) * 255.0 / (hi - lo)), 0, 255).astype(np.uint8)
        q = np.clip(np.round((qx - lo) * 255.0 / (hi - lo)), 0, 255).astype(np.uint8)
    else:
        t = np.float16 if dtype == "f16" else np.float32
        base, q = x.astype(t), qx.astype(t)
    rows = [(qi, ls[0], list(ls), []) for qi, ls in enumerate(wl.query_labels)]
    rs = gp._routeset(rows, li)
    rng = np.random.default_rng(dim + order)
    ids, offs, sizes = _scan_lists(rng, base.shape[0], rs.count)
    dg = gs.DeviceGraph.upload(li)
    dr = gs.DeviceRoutes.upload(rs)
    db = torch.from_numpy(base).cuda()
    dq = torch.from_numpy(q).cuda()
    for with_pred in (False, True):
        pred_o = po.PredicateArrays.from_plan(rs.predicate, li) if with_pred else None
        pv = dr.predicate_view(dg, 0.0, False) if with_pred else None
        for k in (1, 10, 64):
            say("exact posting scan", dtype, "dim", dim, "order", order, "pred", with_pred, "k", k)
            oi, od, op = po.exact_posting_scan(pred_o, base, q, rs.route_query, ids, offs, sizes,
                                               k, order)
            gi_, gd, gp_ = gs.exact_posting(gpu_ctx, db, dq, rs.route_query, ids, offs, sizes, k,
                                            order, pv)
            torch.cuda.synchronize()
            assert np.array_equal(gi_.cpu().numpy().view(np.uint32).reshape(-1, k), oi)
            assert np.array_equal(gd.cpu().numpy().reshape(-1, k).view(np.uint32),
                                  od.view(np.uint32))
            assert np.array_equal(gp_.cpu().numpy().view(np.uint32), op)
            assert (oi[:, 0] != U32MAX).sum() > rs.count // 2


def test_exact_search_invalid_seeds(gpu_ctx, eworld):
    wl, li, rs = eworld
    say("exact search invalid seeds")
    start = rs.route_start.copy()
    start[0] = U32MAX
    start[1] = li.label_size[rs.route_group[1]]
    rs2 = gp.RouteSet(rs.route_query, rs.route_group, start, rs.route_to_query, rs.predicate)
    oi, ost = _run(gpu_ctx, wl, li, rs2, None, lambda dr, dg: _lib.PredicateView(), 32, 10, 2,
                   _lib.PLACE_AUTO, False)
    assert np.all(oi[:2] == U32MAX) and np.all(ost[:2, 0] == 0)


def test_exact_search_rejects_bad_params(gpu_ctx, eworld):
    wl, li, rs = eworld
    dg = gs.DeviceGraph.upload(li)
    dr = gs.DeviceRoutes.upload(rs)
    base, q = wl.base.cuda(), wl.queries.cuda()
    for Q, k, elem in ((1, 10, _lib.ELEM_U8), (32, 11, _lib.ELEM_U8), (32, 10, 3)):
        prm = _lib.ExactParams(Q, 1, 2, 0, k, 0)
        rc = gpu_ctx.lib.gofann_exact_search(gpu_ctx.handle, _lib.ptr(base), elem, wl.dim, wl.n,
                                             _lib.ptr(q), dg.view(), None, _lib.PredicateView(),
                                             dr.routes_view(), prm, None, None, None)
        assert rc in (_lib.ERR_INVALID, _lib.ERR_UNSUPPORTED)
