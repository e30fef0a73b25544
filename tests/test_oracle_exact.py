"""Pins the oracle's full-GPU exact route (run_full_gpu_highfreq_route,
backend_full_gpu.cu:1682-2042) by brute force and by the reference's own
rules: with early stop off and a beam larger than a complete-graph group,
every row of the group is expanded, so the best-k is exactly the k nearest
filter-passing rows by integer squared L2 (ties by sample id); insert_best
keeps a sorted, deduplicated best-k; invalid seeds and out-of-group
adjacency entries are skipped; max_steps and the stats are consistent."""
from __future__ import annotations

import numpy as np
import pytest

import pyoracle as po
from gofann_amd import index as gi
from gofann_amd import plan as gp
from gofann_amd import synth

from test_oracle_search import complete_graph_index

# the index is built by the oracle's restatement of the GPU build (no GPU here)
CPU_BUILD = po.OracleBuild()

U32MAX = 0xFFFFFFFF
FLT_MAX = np.float32(3.4028234663852886e38)


@pytest.fixture(scope="module")
def u8world():
    wl = synth.small_labelled(n=900, nq=12, dim=48, k=6, sigma=0.8, labels=3, seed=15, tags=True,
                              dtype="u8")
    li = gi.build_label_index(wl.base, wl.label_offsets, wl.label_values, wl.num_labels,
                              wl.centroids, degree=24, threshold=50,
                              backend=CPU_BUILD)
    return wl, li


def _l2(base, q):
    return ((base.astype(np.int64) - q.astype(np.int64)) ** 2).sum(-1)


def test_l2_u8_int_is_the_integer_distance():
    rng = np.random.default_rng(0)
    L = po.lib()
    for dim in (1, 3, 16, 48, 192, 1000):
        a = rng.integers(0, 256, dim).astype(np.uint8)
        b = rng.integers(0, 256, dim).astype(np.uint8)
        assert L.orc_l2_u8_int(po.p(a), po.p(b), dim) == int(_l2(a[None], b)[0])


def test_insert_best_matches_sorted_dedup_model():
    """insert_best_result: the best-k is the k least (dist, id) pairs over
    the distinct ids seen, each id at its least distance -- a closed form."""
    rng = np.random.default_rng(1)
    L = po.lib()
    import ctypes as C
    L.orc_insert_best.argtypes = [C.c_float, C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p,
                                  C.POINTER(C.c_uint32)]
    for K in (1, 4, 10):
        bd = np.full(10, FLT_MAX, np.float32)
        bi = np.full(10, U32MAX, np.uint32)
        size = C.c_uint32(0)
        best = {}
        for _ in range(300):
            i = int(rng.integers(0, 40))
            d = float(np.float32(rng.integers(0, 30)))
            L.orc_insert_best(d, i, K, po.p(bd), po.p(bi), C.byref(size))
            best[i] = min(best.get(i, np.inf), d)
        want = sorted((d, i) for i, d in best.items())[:K]
        got = [(float(bd[j]), int(bi[j])) for j in range(size.value)]
        assert got == want


@pytest.mark.parametrize("with_pred", [False, True])
@pytest.mark.parametrize("topk", [1, 5, 10])
def test_exact_full_beam_equals_brute_force(u8world, with_pred, topk):
    wl, _ = u8world
    li = complete_graph_index(wl)
    rs = gp.plan_queries(li, wl.query_labels).graph
    pred = po.PredicateArrays.from_plan(rs.predicate, li) if with_pred else None
    base, q = wl.base.numpy(), wl.queries.numpy()
    ids, dists, st = po.exact_search(li, rs, pred, base, q, queue_limit=1000, topk=topk,
                                     early_stop_mode=1, label_size=li.label_size)
    for r in range(rs.count):
        label, qi = int(rs.route_group[r]), int(rs.route_query[r])
        rows = li.row_to_sample[li.label_offset[label]:li.label_offset[label] + li.label_size[label]]
        allowed = gp.filter_mask(li, wl.query_labels[qi], [], None) if with_pred \
            else np.ones(base.shape[0], bool)
        cand = np.array([s for s in rows if allowed[s]], np.int64)
        d = _l2(base[cand], q[qi]).astype(np.float32)
        want = sorted(zip(d.tolist(), cand.tolist()))[:topk]
        got = [(float(x), int(i)) for x, i in zip(dists[r], ids[r]) if i != U32MAX]
        assert got == want, r
        assert st[r, 1] == li.label_size[label] and st[r, 0] == st[r, 1]   # every row expanded
        assert st[r, 2] == len(cand) and st[r, 7] == 1


def test_exact_route_invalid_seeds_and_group_bounds(u8world):
    wl, li0 = u8world
    li = complete_graph_index(wl)
    rs = gp.plan_queries(li, wl.query_labels).graph
    base, q = wl.base.numpy(), wl.queries.numpy()
    start = rs.route_start.copy()
    start[0] = U32MAX                                  # no seed
    start[1] = li.label_size[rs.route_group[1]]        # seed past the group
    rs.route_start = start
    ids, dists, st = po.exact_search(li, rs, None, base, q, queue_limit=64, topk=10,
                                     label_size=li.label_size)
    for r in (0, 1):
        assert np.all(ids[r] == U32MAX) and np.all(dists[r] == FLT_MAX)
        assert st[r, 0] == 0 and st[r, 7] == 1
    # Adjacency entries at or past the group size are never read as rows.
    g = li.graph.copy()
    g[:, 5] = 10_000_000
    li.graph = g
    ids2, _, _ = po.exact_search(li, rs, None, base, q, queue_limit=64, topk=10,
                                 label_size=li.label_size)
    assert np.all((ids2 == U32MAX) | (ids2 < base.shape[0]))


def test_exact_route_max_steps_and_stats(u8world):
    wl, li = u8world
    rs = gp.plan_queries(li, wl.query_labels).graph
    base, q = wl.base.numpy(), wl.queries.numpy()
    pred = po.PredicateArrays.from_plan(rs.predicate, li)
    for steps in (1, 3, 25):
        ids, dists, st = po.exact_search(li, rs, pred, base, q, queue_limit=32, topk=10,
                                         early_stop_mode=1, max_steps=steps,
                                         label_size=li.label_size)
        assert np.all(st[:, 0] <= steps)
        assert np.all(st[:, 1] == st[:, 0]) and np.all(st[:, 2] <= st[:, 1])
        assert np.all(st[:, 6] <= st[:, 3])
    for mode in (0, 2):
        ids, dists, st = po.exact_search(li, rs, pred, base, q, queue_limit=32, topk=10,
                                         early_stop_mode=mode, label_size=li.label_size)
        for r in range(rs.count):
            got = [(float(x), int(i)) for x, i in zip(dists[r], ids[r]) if i != U32MAX]
            assert got == sorted(got) and len({i for _, i in got}) == len(got)
            qi = int(rs.route_query[r])
            for dd, i in got:
                assert dd == float(_l2(base[i][None], q[qi])[0])


def test_exact_route_legacy_filters(u8world):
    """Row mask & route bits, and every active legacy range, gate the best-k."""
    wl, li = u8world
    li = complete_graph_index(wl)
    rs = gp.plan_queries(li, wl.query_labels).graph
    base, q = wl.base.numpy(), wl.queries.numpy()
    rng = np.random.default_rng(3)
    rows = li.row_to_sample.shape[0]
    rmask = rng.integers(1, 4, rows).astype(np.uint64)          # bits 0/1
    qbits = rng.integers(1, 4, rs.count).astype(np.uint64)
    rc = 2
    brv = rng.integers(0, 10, (base.shape[0], rc)).astype(np.float32)
    modes = rng.integers(0, 4, (rs.count, rc)).astype(np.uint8)
    lo = rng.integers(0, 5, (rs.count, rc)).astype(np.float32)
    hi = lo + rng.integers(2, 8, (rs.count, rc)).astype(np.float32)
    ids, dists, st = po.exact_search(li, rs, None, base, q, queue_limit=1000, topk=10,
                                     early_stop_mode=1, label_size=li.label_size,
                                     row_filter_mask=rmask, query_filter_bits=qbits,
                                     range_modes=modes, range_lower=lo, range_upper=hi,
                                     base_range_values=brv)
    for r in range(rs.count):
        label, qi = int(rs.route_group[r]), int(rs.route_query[r])
        g0, n = int(li.label_offset[label]), int(li.label_size[label])
        ok = []
        for j in range(n):
            s = int(li.row_to_sample[g0 + j])
            if not (int(rmask[g0 + j]) & int(qbits[r])):
                continue
            good = True
            for k in range(rc):
                m, v = int(modes[r, k]), brv[s, k]
                if m == 1:
                    good &= v > lo[r, k]
                elif m == 2:
                    good &= v < hi[r, k]
                elif m == 3:
                    good &= lo[r, k] <= v < hi[r, k]
            if good:
                ok.append(s)
        ok = np.array(ok, np.int64)
        d = _l2(base[ok], q[qi]).astype(np.float32) if ok.size else np.zeros(0, np.float32)
        want = sorted(zip(d.tolist(), ok.tolist()))[:10]
        got = [(float(x), int(i)) for x, i in zip(dists[r], ids[r]) if i != U32MAX]
        assert got == want, r


# ---- float rows: the reference's two summation orders ----------------------

def _int_rows(rng, n, dim, hi=16):
    """Integer-valued rows: every partial sum stays an exact float."""
    return rng.integers(0, hi, (n, dim)).astype(np.int64)


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
@pytest.mark.parametrize("dim", [1, 2, 31, 32, 37, 64, 100, 128, 1000])
def test_float_distances_are_exact_on_integer_rows(dtype, dim):
    """On integer-valued rows every partial sum is exact, so both orders
    equal the integer squared distance: a dropped, repeated or misplaced
    term (a wrong stride, a wrong f16 pair) fails here."""
    rng = np.random.default_rng(dim)
    a, b = _int_rows(rng, 2, dim)
    want = float(((a - b) ** 2).sum())
    for f in (po.l2_w32, po.l2_serial):
        assert f(a.astype(dtype), b.astype(dtype)) == want


def test_w32_tree_known_answer():
    """The halving tree (j, j + 16), (j, j + 8), ... of 32 partials, worked
    by hand: partials 0, 8, 16, 24 hold 2^24, 1, 1, 1.  Tree: (2^24 + 1) ->
    2^24 (ties to even), (1 + 1) = 2, 2^24 + 2 exact -> 16777218.  The
    serial chain adds each 1 to 2^24 and loses it -> 16777216."""
    for dtype in (np.float32, np.float16):
        row = np.zeros(32, dtype)
        row[0], row[8], row[16], row[24] = 4096, 1, 1, 1
        q = np.zeros(32, dtype)
        assert po.l2_w32(row, q) == 16777218.0
        assert po.l2_serial(row, q) == 16777216.0


def test_f16_pair_grouping_known_answer():
    """f16 rows of even dim add each element pair as fma(dx, dx, dy * dy)
    to the running sum.  Partial 0 of a 128-dim row holds pairs 0 and 32:
    (4096, 0) gives 2^24, then (1, 1) adds fma(1, 1, 1) = 2 exactly ->
    16777218 in both orders.  Fusing the running sum into the pair
    (fma(dx, dx, fma(dy, dy, p))) would round 2^24 + 1 twice -> 16777216."""
    row = np.zeros(128, np.float16)
    row[0], row[64], row[65] = 4096, 1, 1
    q = np.zeros(128, np.float16)
    assert po.l2_w32(row, q) == 16777218.0
    assert po.l2_serial(row, q) == 16777218.0
    # odd dim: per element (no pairs): 2^24 + 1 + 1 in the serial chain
    row = np.zeros(67, np.float16)
    row[0], row[64], row[65] = 4096, 1, 1
    assert po.l2_serial(row, np.zeros(67, np.float16)) == 16777216.0


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
@pytest.mark.parametrize("with_pred", [False, True])
def test_exact_full_beam_float_rows_equal_brute_force(u8world, dtype, with_pred):
    """The exact route over f32 / f16 rows (the reference's T = float /
    __half): on integer-valued rows the distances are exact, so a full beam
    over a complete graph returns the brute-force k nearest by (distance,
    id)."""
    wl, _ = u8world
    li = complete_graph_index(wl)
    rs = gp.plan_queries(li, wl.query_labels).graph
    pred = po.PredicateArrays.from_plan(rs.predicate, li) if with_pred else None
    base8, q8 = wl.base.numpy(), wl.queries.numpy()
    base, q = base8.astype(dtype), q8.astype(dtype)
    ids, dists, st = po.exact_search(li, rs, pred, base, q, queue_limit=1000, topk=10,
                                     early_stop_mode=1, label_size=li.label_size)
    i8, d8, s8 = po.exact_search(li, rs, pred, base8, q8, queue_limit=1000, topk=10,
                                 early_stop_mode=1, label_size=li.label_size)
    assert np.array_equal(ids, i8) and np.array_equal(dists, d8) and np.array_equal(st, s8)
    for r in range(rs.count):
        label, qi = int(rs.route_group[r]), int(rs.route_query[r])
        rows = li.row_to_sample[li.label_offset[label]:li.label_offset[label] + li.label_size[label]]
        allowed = gp.filter_mask(li, wl.query_labels[qi], [], None) if with_pred \
            else np.ones(base.shape[0], bool)
        cand = np.array([s for s in rows if allowed[s]], np.int64)
        d = _l2(base8[cand], q8[qi]).astype(np.float32)
        want = sorted(zip(d.tolist(), cand.tolist()))[:10]
        got = [(float(x), int(i)) for x, i in zip(dists[r], ids[r]) if i != U32MAX]
        assert got == want, r


def _posting_lists(rng, n, routes, max_len, dup=True):
    """Random posting lists with duplicates, UINT32_MAX and ids >= n."""
    sizes = rng.integers(0, max_len + 1, routes).astype(np.uint32)
    sizes[0] = 0
    offs = np.zeros(routes, np.uint32)
    offs[1:] = np.cumsum(sizes)[:-1]
    ids = rng.integers(0, n, int(sizes.sum())).astype(np.uint32)
    if dup and len(ids) > 10:
        ids[5:10] = ids[0:5]
        ids[rng.integers(0, len(ids), len(ids) // 20)] = U32MAX
        ids[rng.integers(0, len(ids), len(ids) // 20)] = n + 7
    return ids, offs, sizes


@pytest.mark.parametrize("dtype", [np.uint8, np.float32, np.float16])
@pytest.mark.parametrize("order", [po.EXACT_ORDER_SERIAL, po.EXACT_ORDER_W32])
@pytest.mark.parametrize("with_pred", [False, True])
def test_exact_posting_scan_equals_brute_force(u8world, dtype, order, with_pred):
    """Integer-valued rows: the scan returns the topk distinct listed
    samples by (exact distance, id), skipping UINT32_MAX, ids past the base
    and predicate failures; pass counts count the passing listed entries
    (duplicates included)."""
    wl, li = u8world
    rng = np.random.default_rng(41)
    base8, q8 = wl.base.numpy(), wl.queries.numpy()
    base, q = base8.astype(dtype), q8.astype(dtype)
    # one route per query; its predicate is every label of the query
    rows = [(qi, ls[0], list(ls), []) for qi, ls in enumerate(wl.query_labels)]
    rs = gp._routeset(rows, li)
    R = rs.count
    ids, offs, sizes = _posting_lists(rng, base.shape[0], R, 300)
    pred = po.PredicateArrays.from_plan(rs.predicate, li) if with_pred else None
    for k in (1, 10, 64):
        oi, od, op = po.exact_posting_scan(pred, base, q, rs.route_query, ids, offs, sizes, k,
                                           order)
        for r in range(R):
            qi = int(rs.route_query[r])
            allowed = gp.filter_mask(li, wl.query_labels[qi], [], None) if with_pred \
                else np.ones(base.shape[0], bool)
            lst = ids[offs[r]:offs[r] + sizes[r]].astype(np.int64)
            ok = [int(s) for s in lst if s < base.shape[0] and allowed[s]]
            assert op[r] == len(ok)
            uniq = np.array(sorted(set(ok)), np.int64)
            d = _l2(base8[uniq], q8[qi]).astype(np.float32) if len(uniq) else np.zeros(0)
            want = sorted(zip(d.tolist(), uniq.tolist()))[:k]
            got = [(float(x), int(i)) for x, i in zip(od[r], oi[r]) if i != U32MAX]
            assert got == want, (r, k)
            assert np.all(oi[r, len(want):] == U32MAX) and np.all(od[r, len(want):] == FLT_MAX)


def test_exact_posting_scan_order_changes_ties():
    """Row 0 scores 16777218 in the warp order and 16777216 in the serial
    order (the known answer above); row 1 scores 16777216 in both.  The
    serial scan ranks row 0 first (tie, smaller id), the warp scan row 1."""
    base = np.zeros((2, 32), np.float32)
    base[0, [0, 8, 16, 24]] = 4096, 1, 1, 1
    base[1, 0] = 4096
    q = np.zeros((1, 32), np.float32)
    args = (None, base, q, [0], [0, 1], [0], [2], 1)
    assert po.exact_posting_scan(*args, po.EXACT_ORDER_SERIAL)[0][0, 0] == 0
    assert po.exact_posting_scan(*args, po.EXACT_ORDER_W32)[0][0, 0] == 1
