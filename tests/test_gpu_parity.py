"""GPU parity: the HIP kernels, called through the C ABI, against the CPU
oracle on the same seeded inputs.  Integer, index and ordering outputs must
be identical; floats are compared bit for bit where the kernel reproduces
the oracle's operation order (traversal, posting scans, rerank) and with the
reference's own tolerances where a GEMM order differs (RaBitQ rotation and
centroid distances: rabitq_query_rotation_test.cu:31, 47-49)."""
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


def as_u32(t: torch.Tensor) -> np.ndarray:
    return t.cpu().numpy().view(np.uint32)


@pytest.fixture(scope="module", params=["u8-tags", "f32-labels", "f32-ranges"])
def world(request):
    kind = request.param
    if kind == "u8-tags":
        wl = synth.small_labelled(n=6000, nq=48, dim=48, k=12, sigma=0.7, labels=7, seed=21,
                                  dtype="u8", tags=True)
    elif kind == "f32-labels":
        wl = synth.small_labelled(n=6000, nq=48, dim=64, k=12, sigma=0.7, labels=5, seed=22)
    else:
        wl = synth.small_labelled(n=6000, nq=48, dim=32, k=12, sigma=0.7, labels=4, seed=23,
                                  tags=True, ranges=True)
    li = gi.build_label_index(wl.base, wl.label_offsets, wl.label_values, wl.num_labels,
                              wl.centroids, degree=32, threshold=300)
    pl = gp.plan_queries(li, wl.query_labels, wl.query_ranges)
    return kind, wl, li, pl


def _pq(wl, M):
    table = gi.train_pq(wl.base, M, iters=6)
    codes = gi.pq_encode(wl.base, table, M)
    return table, codes


# Placements of the per-route state: (ADC table, visited set, neighbour
# sample table, sample records: codes + inline label slab, "overflow" forcing
# every third row onto the CSR).  Every placement must give the oracle's bits.
PLACEMENTS = {
    "auto": (_lib.PLACE_AUTO, _lib.PLACE_AUTO, False, None),
    "lds-lds-nsamp": (_lib.PLACE_LDS, _lib.PLACE_LDS, True, None),
    "direct-global-nsamp": (_lib.PLACE_GLOBAL, _lib.PLACE_GLOBAL, True, None),
    "direct-lds": (_lib.PLACE_GLOBAL, _lib.PLACE_LDS, False, None),
    "direct-spill-nsamp": (_lib.PLACE_GLOBAL, _lib.PLACE_SPILL, True, None),
    "lds-spill": (_lib.PLACE_LDS, _lib.PLACE_SPILL, False, None),
    "auto-records": (_lib.PLACE_AUTO, _lib.PLACE_AUTO, True, "slab"),
    "lds-records-overflow": (_lib.PLACE_LDS, _lib.PLACE_GLOBAL, False, "overflow"),
}


def records_for(codes, li, kind):
    if kind is None:
        return None
    return gs.SampleRecords.build(codes, li.csr_offsets, li.csr_labels,
                                  overflow_every=3 if kind == "overflow" else 0)
HASH_CODE = {_lib.PLACE_GLOBAL: 0, _lib.PLACE_LDS: 1, _lib.PLACE_SPILL: 2}


@pytest.mark.parametrize("place", list(PLACEMENTS))
@pytest.mark.parametrize("M", [16, 32, 48])
@pytest.mark.parametrize("mode", ["adaptive-bias", "off", "fixed-nobias"])
def test_pq_search_matches_oracle(gpu_ctx, world, M, mode, place):
    kind, wl, li, pl = world
    if wl.dim % M:
        pytest.skip("pq_dim must divide dim")
    table_mode, hash_mode, nsamp, rec = PLACEMENTS[place]
    say("pq_search", kind, M, mode, place)
    table, codes = _pq(wl, M)
    rs = pl.graph
    bias = mode == "adaptive-bias"
    es = {"adaptive-bias": 2, "off": 1, "fixed-nobias": 0}[mode]
    Q, W = (48, 40) if mode != "off" else (24, 16)
    maxs = 60 if mode == "off" else 0
    pred_o = po.PredicateArrays.from_plan(rs.predicate, li, wl.base_ranges, alpha=0.15 if bias else 0.0,
                                          pending_base_stop=bias)
    prm_o = po.params(queue_limit=Q, result_width=W, early_stop_mode=es, finish_limit=3,
                      max_steps=maxs, bias=bias)
    q = wl.queries.numpy()
    oi, od, ost = po.pq_search(li, rs, pred_o, prm_o, codes.numpy(), table.numpy(), q)

    dg = gs.DeviceGraph.upload(li, neighbor_samples=nsamp)
    dr = gs.DeviceRoutes.upload(rs, wl.base_ranges)
    records = records_for(codes, li, rec)
    keep = (records if records is not None else codes.cuda(), table.cuda())
    pqv = gs.pq_view(*keep)
    qd = wl.queries.cuda()
    prm = gs.search_params(queue_limit=Q, result_width=W, early_stop_mode=es, finish_limit=3,
                           max_steps=maxs, bias=bias, table_mode=table_mode, hash_mode=hash_mode)
    ids, dists, st = gs.run_pq_routes(gpu_ctx, pqv, qd, dg, dr, prm,
                                      alpha=0.15 if bias else 0.0, pending_base_stop=bias,
                                      records=records)
    torch.cuda.synchronize()
    gi_ = as_u32(ids).reshape(rs.count, W)
    gd = dists.cpu().numpy().reshape(rs.count, W)
    gst = st.cpu().numpy().reshape(rs.count, 8)
    placed = gpu_ctx.last_placement()
    say("routes", rs.count, placed)
    if table_mode != _lib.PLACE_AUTO:
        assert placed["table_in_lds"] == (1 if table_mode == _lib.PLACE_LDS else 0)
        assert placed["hash_in_lds"] == HASH_CODE[hash_mode]
    assert np.array_equal(gi_, oi), "route ids differ"
    assert np.array_equal(gd.view(np.uint32), od.view(np.uint32)), "distances differ in bits"
    assert np.array_equal(gst, ost), "per-route counters differ"


@pytest.mark.parametrize("place", list(PLACEMENTS))
@pytest.mark.parametrize("W", [10, 40])
def test_pq_search_inline_exact_matches_oracle(gpu_ctx, world, W, place):
    """Inline exact distances (enable_true_distance_rerank) on resident
    vectors: identical ids, distance bits and counters."""
    kind, wl, li, pl = world
    table_mode, hash_mode, nsamp, rec = PLACEMENTS[place]
    say("pq_search inline exact", kind, W, place)
    table, codes = _pq(wl, 16)
    rs = pl.graph
    pred_o = po.PredicateArrays.from_plan(rs.predicate, li, wl.base_ranges, alpha=0.15,
                                          pending_base_stop=True)
    prm_o = po.params(queue_limit=48, result_width=W, inline_exact=True)
    base = wl.base.numpy()
    oi, od, ost = po.pq_search(li, rs, pred_o, prm_o, codes.numpy(), table.numpy(),
                               wl.queries.numpy(), base=base)
    dg = gs.DeviceGraph.upload(li, neighbor_samples=nsamp)
    dr = gs.DeviceRoutes.upload(rs, wl.base_ranges)
    records = records_for(codes, li, rec)
    keep = (records if records is not None else codes.cuda(), table.cuda(), wl.base.cuda())
    pqv = gs.pq_view(*keep)
    prm = gs.search_params(queue_limit=48, result_width=W, inline_exact=True,
                           table_mode=table_mode, hash_mode=hash_mode)
    ids, dists, st = gs.run_pq_routes(gpu_ctx, pqv, wl.queries.cuda(), dg, dr, prm,
                                      records=records)
    torch.cuda.synchronize()
    assert np.array_equal(as_u32(ids).reshape(rs.count, W), oi)
    assert np.array_equal(dists.cpu().numpy().reshape(rs.count, W).view(np.uint32),
                          od.view(np.uint32))
    assert np.array_equal(st.cpu().numpy().reshape(rs.count, 8), ost)
    # results are exact squared distances
    for r in range(min(rs.count, 8)):
        q = wl.queries.numpy()[rs.route_query[r]].astype(np.float64)
        for i, d in zip(oi[r], od[r]):
            if i != U32MAX:
                assert abs(((base[i].astype(np.float64) - q) ** 2).sum() - d) <= 1e-5 * max(1.0, d)


# ---- the shapes the benches launch: C2 (dim 192, u8, PQ M = 48, degree 64,
# tags: traversal_kernel<PqScorer<48, 4>>) and C1 (dim 128, f32, PQ M = 32,
# degree 32, ten labels: PqScorer<32, 4>).  Graphs are bucketed by trained
# k-means centres and searched from each label's medoid, as the benches do.
BENCH_SHAPES = {
    "c2-shape": dict(dim=192, M=48, degree=64, dtype="u8", tags=True, labels=6, seed=24),
    "c1-shape": dict(dim=128, M=32, degree=32, dtype="f32", tags=False, labels=10, seed=25),
}


@pytest.fixture(scope="module", params=list(BENCH_SHAPES))
def bench_world(request):
    cfg = BENCH_SHAPES[request.param]
    wl = synth.small_labelled(n=9000, nq=40, dim=cfg["dim"], k=14, sigma=0.7,
                              labels=cfg["labels"], seed=cfg["seed"], dtype=cfg["dtype"],
                              tags=cfg["tags"])
    cen = gi.train_kmeans(wl.base, 14, seed=cfg["seed"])
    li = gi.build_label_index(wl.base, wl.label_offsets, wl.label_values, wl.num_labels, cen,
                              degree=cfg["degree"], threshold=300)
    pl = gp.plan_queries(li, wl.query_labels)
    table, codes = _pq(wl, cfg["M"])
    return request.param, cfg, wl, li, pl, table, codes


BENCH_PLACES = ["auto", "lds-lds-nsamp", "direct-spill-nsamp", "direct-global-nsamp",
                "auto-records", "lds-records-overflow"]


@pytest.mark.parametrize("place", BENCH_PLACES)
@pytest.mark.parametrize("mode", ["adaptive-bias", "inline-exact", "fixed-nobias"])
def test_pq_search_bench_shapes_match_oracle(gpu_ctx, bench_world, place, mode):
    kind, cfg, wl, li, pl, table, codes = bench_world
    table_mode, hash_mode, nsamp, rec = PLACEMENTS[place]
    say("pq_search bench shape", kind, mode, place)
    rs = pl.graph
    inline = mode == "inline-exact"
    bias = mode != "fixed-nobias"
    Q, W = (64, 10) if inline else (96, 100)
    es = 0 if mode == "fixed-nobias" else 2
    pred_o = po.PredicateArrays.from_plan(rs.predicate, li, alpha=0.15 if bias else 0.0,
                                          pending_base_stop=bias)
    prm_o = po.params(queue_limit=Q, result_width=W, early_stop_mode=es, finish_limit=3,
                      bias=bias, inline_exact=inline)
    base = wl.base.numpy()
    oi, od, ost = po.pq_search(li, rs, pred_o, prm_o, codes.numpy(), table.numpy(),
                               wl.queries.numpy(), base=base if inline else None)
    dg = gs.DeviceGraph.upload(li, neighbor_samples=nsamp)
    dr = gs.DeviceRoutes.upload(rs)
    records = records_for(codes, li, rec)
    keep = (records if records is not None else codes.cuda(), table.cuda()) + \
        ((wl.base.cuda(),) if inline else ())
    prm = gs.search_params(queue_limit=Q, result_width=W, early_stop_mode=es, finish_limit=3,
                           bias=bias, inline_exact=inline, table_mode=table_mode,
                           hash_mode=hash_mode)
    ids, dists, st = gs.run_pq_routes(gpu_ctx, gs.pq_view(*keep), wl.queries.cuda(), dg, dr, prm,
                                      alpha=0.15 if bias else 0.0, pending_base_stop=bias,
                                      records=records)
    torch.cuda.synchronize()
    say("routes", rs.count, gpu_ctx.last_placement())
    assert np.array_equal(as_u32(ids).reshape(rs.count, W), oi), "route ids differ"
    assert np.array_equal(dists.cpu().numpy().reshape(rs.count, W).view(np.uint32),
                          od.view(np.uint32)), "distances differ in bits"
    assert np.array_equal(st.cpu().numpy().reshape(rs.count, 8), ost), "counters differ"
    assert (oi[:, 0] != U32MAX).sum() > rs.count // 2
    if cfg["degree"] == 64:
        # lanes 32..63 of the adjacency row carry live neighbours
        assert (li.graph[:, 32:] != U32MAX).any(1).mean() > 0.5


@pytest.fixture(scope="module")
def long_world():
    """One 12k-row label graph, degree 64, and PQ codes that are all zero:
    every candidate ties, so a beam without early stop admits far more than
    the visited set's 4096 values (it fills and drops), and the spilling
    LDS table moves to its global slab early."""
    wl = synth.small_labelled(n=12000, nq=6, dim=32, k=8, sigma=1.0, labels=1, seed=32)
    li = gi.build_label_index(wl.base, wl.label_offsets, wl.label_values, wl.num_labels,
                              wl.centroids, degree=64, threshold=300)
    pl = gp.plan_queries(li, wl.query_labels)
    table = gi.train_pq(wl.base, 8, iters=3)
    codes = torch.zeros(wl.n, 8, dtype=torch.uint8)
    return wl, li, pl, table, codes


@pytest.mark.parametrize("place", list(PLACEMENTS))
# all-tie frontiers of 258 and 402 slots (past 260, pairs 64.. have children);
# 602 slots: past the wave-parallel frontier's 512, the serial lane-0 sifts
@pytest.mark.parametrize("Q", [256, 400, 600])
def test_pq_search_visited_fill_matches_oracle(gpu_ctx, long_world, place, Q):
    wl, li, pl, table, codes = long_world
    table_mode, hash_mode, nsamp, rec = PLACEMENTS[place]
    say("pq_search visited fill", place, "Q", Q)
    rs = pl.graph
    W, steps = 40, 450
    pred_o = po.PredicateArrays.from_plan(rs.predicate, li, alpha=0.0, pending_base_stop=False)
    prm_o = po.params(queue_limit=Q, result_width=W, early_stop_mode=1, max_steps=steps,
                      bias=False)
    oi, od, ost = po.pq_search(li, rs, pred_o, prm_o, codes.numpy(), table.numpy(),
                               wl.queries.numpy())
    assert ost[:, 6].max() > 4096, "the beam must overfill the visited set"
    dg = gs.DeviceGraph.upload(li, neighbor_samples=nsamp)
    dr = gs.DeviceRoutes.upload(rs)
    records = records_for(codes, li, rec)
    keep = (records if records is not None else codes.cuda(), table.cuda())
    prm = gs.search_params(queue_limit=Q, result_width=W, early_stop_mode=1, max_steps=steps,
                           bias=False, table_mode=table_mode, hash_mode=hash_mode)
    ids, dists, st = gs.run_pq_routes(gpu_ctx, gs.pq_view(*keep), wl.queries.cuda(), dg, dr, prm,
                                      alpha=0.0, pending_base_stop=False, records=records)
    torch.cuda.synchronize()
    assert np.array_equal(as_u32(ids).reshape(rs.count, W), oi)
    assert np.array_equal(dists.cpu().numpy().reshape(rs.count, W).view(np.uint32),
                          od.view(np.uint32))
    assert np.array_equal(st.cpu().numpy().reshape(rs.count, 8), ost)


def test_pq_search_batched_launch_order(gpu_ctx, world):
    """Route sub-ranges and the XCD slot mapping give the same answers."""
    kind, wl, li, pl = world
    say("pq_search batches", kind)
    table, codes = _pq(wl, 16)
    rs = pl.graph
    dg = gs.DeviceGraph.upload(li)
    dr = gs.DeviceRoutes.upload(rs, wl.base_ranges)
    keep = (codes.cuda(), table.cuda())
    pqv = gs.pq_view(*keep)
    qd = wl.queries.cuda()
    prm = gs.search_params(queue_limit=32, result_width=20)
    a = gs.run_pq_routes(gpu_ctx, pqv, qd, dg, dr, prm)
    n = rs.count
    out = (torch.empty_like(a[0]), torch.empty_like(a[1]), torch.zeros_like(a[2]))
    for b0 in range(0, n, 7):
        gs.run_pq_routes(gpu_ctx, pqv, qd, dg, dr, prm, begin=b0, end=min(n, b0 + 7), out=out)
    torch.cuda.synchronize()
    assert torch.equal(a[0], out[0]) and torch.equal(a[1], out[1]) and torch.equal(a[2], out[2])


def test_pq_score_matches_oracle_adc(gpu_ctx, world):
    kind, wl, li, pl = world
    say("pq_score", kind)
    M = 16
    table, codes = _pq(wl, M)
    rng = np.random.default_rng(1)
    n = 500
    qi = np.sort(rng.integers(0, wl.queries.shape[0], n)).astype(np.uint32)
    si = rng.integers(0, wl.n, n).astype(np.uint32)
    keep = (codes.cuda(), table.cuda())
    pqv = gs.pq_view(*keep)
    qd = wl.queries.cuda()
    out = torch.empty(n, dtype=torch.float32, device="cuda")
    qt, st = gs.u32(qi), gs.u32(si)
    gpu_ctx.check(gpu_ctx.lib.gofann_pq_score(gpu_ctx.handle, pqv, _lib.ptr(qd), gs.query_elem(qd),
                                              _lib.ptr(qt), _lib.ptr(st), n, _lib.ptr(out)))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    q = wl.queries.numpy()
    want = np.array([po.pq_adc(po.pq_lut(table.numpy(), q[a], M), codes.numpy()[b])
                     for a, b in zip(qi, si)], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_predicate_masks_fixture(gpu_ctx):
    """gpu_predicate_parallel_test.cu: ballot masks equal scalar matches for
    counts {0, 1, 17, 31, 32, 33, 63, 64, 65, 97}, partial words zero."""
    say("predicate masks")
    fx = load_golden("predicate_parallel.json")
    from gofann_amd.plan import CLAUSE_DTYPE, RANGE_DTYPE
    clauses = np.array([tuple(c) for c in fx["clauses"]], dtype=CLAUSE_DTYPE)
    ranges = np.array([tuple(r) for r in fx["ranges"]], dtype=RANGE_DTYPE)
    pa = po.PredicateArrays(fx["route_offsets"], fx["handles"], clauses, ranges,
                            fx["route_enabled"], None, fx["csr_offsets"], fx["csr_labels"],
                            fx["rows"], np.array(fx["base_ranges"], np.float32))
    import ctypes as C
    L = po.lib()
    dev = {k: gs.to_dev(v) for k, v in [("off", np.array(fx["route_offsets"], np.uint32)),
                                         ("h", np.array(fx["handles"], np.uint32)),
                                         ("cl", clauses), ("rg", ranges),
                                         ("en", np.array(fx["route_enabled"], np.uint8)),
                                         ("br", np.array(fx["base_ranges"], np.float32)),
                                         ("co", np.array(fx["csr_offsets"], np.uint32)),
                                         ("cv", np.array(fx["csr_labels"], np.uint32))]}
    pv = _lib.PredicateView(*[_lib.ptr(dev[k]) for k in ("off", "h", "cl", "rg", "en")], None,
                            _lib.ptr(dev["br"]), _lib.ptr(dev["co"]), _lib.ptr(dev["cv"]),
                            fx["rows"], 2, 0.0, 0)
    mapping = np.array(fx["mapping"], np.uint32)
    for route in range(len(fx["route_enabled"])):
        for count in fx["counts"]:
            samples = np.array([mapping[fx["offset"] + (i * 37) % 97] for i in range(count)],
                               np.uint32)
            routes = np.full(count, route, np.uint32)
            words = (count + 31) // 32
            masks = torch.full((max(words, 1),), -559038737, dtype=torch.int32, device="cuda")
            rt, stt = gs.u32(routes if count else np.zeros(1, np.uint32)), \
                gs.u32(samples if count else np.zeros(1, np.uint32))
            gpu_ctx.check(gpu_ctx.lib.gofann_predicate_masks(gpu_ctx.handle, pv, _lib.ptr(rt),
                                                             _lib.ptr(stt), count, _lib.ptr(masks)))
            torch.cuda.synchronize()
            m = as_u32(masks)
            for i in range(count):
                want = L.orc_pred_enabled(C.byref(pa.struct), route) and \
                    L.orc_pred_matches(C.byref(pa.struct), route, int(samples[i]), None)
                assert bool((m[i // 32] >> (i % 32)) & 1) == bool(want), (route, count, i)
            if count % 32:
                assert (m[count // 32] >> (count % 32)) == 0
            if count == 0:
                assert m[0] == np.uint32(0xDEADBEEF)


def test_pq_posting_scan_matches_oracle(gpu_ctx, world):
    kind, wl, li, pl = world
    say("pq posting scan", kind)
    M = 16
    table, codes = _pq(wl, M)
    # scan every label's posting as a route (routes of all queries x labels)
    labels = wl.query_labels
    rows = []
    for qi, ls in enumerate(labels):
        anchor = ls[0]
        rows.append((qi, anchor, [l for l in ls if l != anchor],
                     [tuple(a) for a in (wl.query_ranges[qi] if wl.query_ranges else [])]))
    rs = gp._routeset(rows, li)
    off = np.array([li.posting_offset[r[1]] for r in rows], np.uint32)
    size = np.array([li.posting_offset[r[1] + 1] - li.posting_offset[r[1]] for r in rows], np.uint32)
    for k in (10, 100, 257):
        pred = po.PredicateArrays.from_plan(rs.predicate, li, wl.base_ranges)
        oi, od, opass = po.posting_scan_pq(pred, codes.numpy(), table.numpy(), wl.queries.numpy(),
                                           rs.route_query, li.posting_ids, off, size, k)
        dg = gs.DeviceGraph.upload(li)
        dr = gs.DeviceRoutes.upload(rs, wl.base_ranges)
        keep = (codes.cuda(), table.cuda())
        pqv = gs.pq_view(*keep)
        ids, dists, passes = gs.run_pq_posting(gpu_ctx, pqv, wl.queries.cuda(), dg, dr, off, size, k)
        torch.cuda.synchronize()
        assert np.array_equal(as_u32(ids).reshape(-1, k), oi)
        assert np.array_equal(dists.cpu().numpy().reshape(-1, k).view(np.uint32), od.view(np.uint32))
        assert np.array_equal(as_u32(passes), opass)


# dim 72 stays in the per-element tail; 1100 and 4096 run the batched loads
# (16 elements a lane) and, for 1100, a tail after them.
@pytest.mark.parametrize("d", [72, 1100, 4096])
@pytest.mark.parametrize("elem", ["u8", "f32", "f16"])
def test_exact_rerank_matches_oracle(gpu_ctx, elem, d):
    say("rerank", elem, "dim", d)
    rng = np.random.default_rng(5)
    n, routes, width, topk = 2000, 40, 100, 10
    if elem == "u8":
        base = rng.integers(0, 256, (n, d)).astype(np.uint8)
        q = rng.integers(0, 256, (routes, d)).astype(np.uint8)
    else:
        base = rng.normal(size=(n, d)).astype(np.float32 if elem == "f32" else np.float16)
        q = rng.normal(size=(routes, d)).astype(np.float32)
    sl = rng.integers(0, n + 10, (routes, width)).astype(np.uint32)
    sl[:, ::11] = U32MAX
    sl[:, 3] = sl[:, 4]
    rq = np.arange(routes, dtype=np.uint32)
    oi, od = po.rerank(base, q, rq, sl, topk)
    bt = torch.from_numpy(base).cuda()
    ids, dists = gs.exact_rerank(gpu_ctx, bt, torch.from_numpy(q).cuda(), gs.u32(rq), gs.u32(sl),
                                 width, routes, topk)
    torch.cuda.synchronize()
    assert np.array_equal(as_u32(ids).reshape(routes, topk), oi)
    assert np.array_equal(dists.cpu().numpy().reshape(routes, topk).view(np.uint32), od.view(np.uint32))


def test_merge_routes_matches_oracle(gpu_ctx):
    say("merge routes")
    fx = load_golden("route_merge.json")
    rng = np.random.default_rng(9)
    cases = [(np.array(c["route_to_query"], np.uint32), np.array(c["ids"], np.uint32),
              np.array(c["dists"], np.float32), c["queries"], c["topk"], c["expected"])
             for c in fx["cases"]]
    for _ in range(6):
        routes, width, queries, topk = int(rng.integers(1, 300)), int(rng.integers(1, 20)), \
            int(rng.integers(1, 60)), int(rng.integers(1, 12))
        ids = rng.integers(0, 50, (routes, width)).astype(np.uint32)
        ids[rng.random((routes, width)) < 0.2] = U32MAX
        d = (rng.integers(0, 40, (routes, width)) / 4).astype(np.float32)
        cases.append((rng.integers(0, queries, routes).astype(np.uint32), ids, d, queries, topk, None))
    for r2q, ids, d, queries, topk, expected in cases:
        oi, od = po.merge(r2q, ids, d, queries, topk)
        if expected is not None:
            assert oi.tolist() == expected
        off, order = gs.query_route_csr(r2q, queries)
        gi_, gd = gs.merge_routes_gpu(gpu_ctx, gs.u32(off), gs.u32(order), gs.u32(ids.reshape(-1)),
                                      gs.to_dev(d.reshape(-1)), ids.shape[1], queries, topk)
        torch.cuda.synchronize()
        assert np.array_equal(as_u32(gi_).reshape(queries, topk), oi)
        assert np.array_equal(gd.cpu().numpy().reshape(queries, topk).view(np.uint32), od.view(np.uint32))


@pytest.mark.parametrize("chunk", [7, 1000])
def test_pq_search_streamed_host_rerank(gpu_ctx, world, chunk):
    """Chunked GPU traversal with the shortlist streamed through pinned host
    memory to the CPU rerank pool equals one traversal launch followed by
    the same rerank, and its shortlists equal the oracle's."""
    kind, wl, li, pl = world
    say("streamed host rerank", kind, chunk)
    table, codes = _pq(wl, 16)
    rs = pl.graph
    W, topk = 40, 10
    dg = gs.DeviceGraph.upload(li)
    dr = gs.DeviceRoutes.upload(rs, wl.base_ranges)
    keep = (codes.cuda(), table.cuda())
    pqv = gs.pq_view(*keep)
    prm = gs.search_params(queue_limit=48, result_width=W)
    ids, dists, st = gs.run_pq_routes(gpu_ctx, pqv, wl.queries.cuda(), dg, dr, prm)
    torch.cuda.synchronize()
    shortlist = as_u32(ids).reshape(rs.count, W)
    pred_o = po.PredicateArrays.from_plan(rs.predicate, li, wl.base_ranges, alpha=0.15,
                                          pending_base_stop=True)
    oi, _, _ = po.pq_search(li, rs, pred_o, po.params(queue_limit=48, result_width=W),
                            codes.numpy(), table.numpy(), wl.queries.numpy())
    assert np.array_equal(shortlist, oi)
    base = wl.base.numpy()
    hr = gs.HostRerank(base, wl.queries.numpy(), threads=4)
    ri, rd = hr.rerank(shortlist, rs.route_query, topk)
    st2 = torch.zeros_like(st)
    si, sd = hr.search(gpu_ctx, pqv, wl.queries.cuda(), dg, dr, prm, rs.route_query, chunk, topk,
                       stats=st2)
    hr.close()
    assert np.array_equal(si, ri)
    assert np.array_equal(sd.view(np.uint32), rd.view(np.uint32))
    assert torch.equal(st, st2)
